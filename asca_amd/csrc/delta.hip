// Gated delta rule, recurrent form, f32, for gfx950.
//
// Math (per sequence b, head h; S is dh x dh, S_0 = 0), as in
// rust/src/delta.rs:1-14 and DeltaBlock::scan_cpu (rust/src/delta.rs:244-334):
//   sk_t = S_{t-1}^T k_t,  u_t = beta_t (v_t - alpha_t sk_t),
//   S_t  = alpha_t S_{t-1} + k_t u_t^T,  o_t = S_t^T q_t.
//
// Design (MI355X-first, not a translation of rust/kernels/asca.cu):
//  * Column i of S only ever meets k, q, alpha, beta and its own v_i, sk_i, u_i,
//    so the forward splits each (sequence, head) unit into dh/8 waves of 8 value
//    columns that never talk to each other (two waves per SIMD at dh = 64).
//    Inside a wave, lane = 8*column + part; a lane keeps dh/8 rows of its column
//    in VGPRs and S^T k, S^T q are 8-lane DPP butterflies.  The k, q rows and v columns of each C-step chunk are staged
//    once per unit in LDS (double-buffered, loaded one chunk ahead, one barrier
//    per chunk) because per-lane global loads of the replicated rows saturate
//    the texture-address path; the step loop is straight-line (unrolled per
//    chunk), the gates of a chunk arrive as one lane-distributed load and are
//    broadcast with v_readlane, outputs of 8 steps leave in one store per lane,
//    and masked lanes store into a trash buffer instead of branching.
//  * The forward stores S every C steps ("checkpoints", C = 8 at dh = 64, laid
//    out as S^T so each lane writes 16-byte vectors) and the per-step sk vector,
//    instead of the reference's full (T+1) dh^2 history (2.15 GB at B32 T512 H8
//    dh64).
//  * The backward walks C-step segments in reverse on dh/8 waves per unit (two
//    per SIMD at dh = 64, so one wave's LDS/scalar work issues beside the
//    other's VALU work).  Each segment's inputs are staged in LDS (loaded one
//    segment ahead, double-buffered), the segment is recomputed from its
//    checkpoint into registers, then processed backwards.  A lane owns a
//    (dh/16) x 2 tile: du = dS^T k is a 16-lane DPP butterfly inside a row,
//    the column sums of dq and dk are transposed permlane32/permlane16 swaps
//    plus a per-segment cross-wave sum through LDS, where the L2-norm and
//    sigmoid backward of the drop-in variant also run.
#include "common.h"
#include "delta.h"
#include "runtime.h"

namespace asca {

template <int DH>
struct DS {
    static constexpr int W = DH / 16;        // waves per unit, 16 value columns each
    static constexpr int THREADS = 64 * W;
    static constexpr int R = DH / 4;         // forward: rows per lane (4 lanes / column)
    // Checkpoint interval C (forward chunk = backward segment).
    static constexpr int CK = (DH == 128) ? 2 : 8;
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
//
// Shape of the forward: a unit runs on DH/8 waves (two per SIMD at dh = 64),
// each owning 8 value columns.  Lane = 8*column + part; a lane keeps rows
// part*R .. part*R+R-1 (R = DH/8) of its column, so S^T k and S^T q are 8-lane
// DPP butterflies (quad_perm, row_half_mirror).

// CS: the unit's value columns are split over CS blocks (1 or 2); each block
// runs W waves of 8 columns.
template <int DH, int CS = 1>
struct FS {
    static constexpr int W = DH / 8 / CS;
    static constexpr int NT = 64 * W;
    static constexpr int R = DH / 8;
    static constexpr int CK = DS<DH>::CK;
    static constexpr int G = CK < 8 ? CK : 8;                 // steps per batched output store
    // LDS: two chunk buffers, each the k and q rows of CK steps (shared by the
    // unit's waves) and every wave's 8 v columns
    static constexpr int KQ_F = CK * DH;
    static constexpr int V_F = W * CK * 8;
    static constexpr int BUF_F = 2 * KQ_F + V_F;
    static constexpr int NKQ = (2 * KQ_F / 4 + NT - 1) / NT;  // staged k/q float4 per thread
    static constexpr int NV = (CK * 2 + 63) / 64;             // staged v float4 per lane
};

template <int DH, int CS>
struct FwdStage {
    float4 kq[FS<DH, CS>::NKQ];
    float4 v[FS<DH, CS>::NV];
};

// Global -> registers for chunk c (steps c*CK .. c*CK+CK-1, clamped to T-1);
// wg: the wave's index among all waves of the unit (its value columns).
template <int DH, int CS, bool EXACT>
ASCA_DEV void fwd_stage_load(FwdStage<DH, CS>& st, int c, const float* __restrict__ q, const float* __restrict__ k,
                             const float* __restrict__ v, long ubase, long d, int T, int dh, int wg, int lane) {
    using L = FS<DH, CS>;
    constexpr int CK = L::CK;
    const int t0 = c * CK;
#pragma unroll
    for (int i = 0; i < L::NKQ; ++i) {
        const int f0 = (int)threadIdx.x + i * L::NT;
        const int f = f0 < L::KQ_F / 2 ? f0 : 0;
        const int tsr = f >= L::KQ_F / 4;
        const int fl = f - tsr * (L::KQ_F / 4);
        const int j = fl / (DH / 4), c4 = fl % (DH / 4);
        const long t = min(t0 + j, T - 1);
        st.kq[i] = ld4m<EXACT>((tsr ? q : k) + ubase + t * d, 4 * c4, dh);
    }
#pragma unroll
    for (int i = 0; i < L::NV; ++i) {
        const int f0 = lane + 64 * i;
        const int f = f0 < CK * 2 ? f0 : 0;
        const int j = f / 2, half = f % 2;
        const long t = min(t0 + j, T - 1);
        st.v[i] = ld4m<EXACT>(v + ubase + t * d, wg * 8 + half * 4, dh);
    }
}

template <int DH, int CS>
ASCA_DEV void fwd_stage_store(const FwdStage<DH, CS>& st, float* __restrict__ buf, int w, int lane) {
    using L = FS<DH, CS>;
    constexpr int CK = L::CK;
#pragma unroll
    for (int i = 0; i < L::NKQ; ++i) {
        const int f = (int)threadIdx.x + i * L::NT;
        if (f < L::KQ_F / 2) {
            const int tsr = f >= L::KQ_F / 4;
            const int fl = f - tsr * (L::KQ_F / 4);
            const int j = fl / (DH / 4), c4 = fl % (DH / 4);
            *reinterpret_cast<float4*>(buf + tsr * L::KQ_F + j * DH + 4 * c4) = st.kq[i];
        }
    }
#pragma unroll
    for (int i = 0; i < L::NV; ++i) {
        const int f = lane + 64 * i;
        if (f < CK * 2) {
            const int j = f / 2, half = f % 2;
            *reinterpret_cast<float4*>(buf + 2 * L::KQ_F + (w * CK + j) * 8 + half * 4) = st.v[i];
        }
    }
}

// LDS -> registers: the k, q rows and the v value one lane needs for step jj.
template <int DH>
ASCA_DEV void fwd_rd(float (&kk)[DH / 8], float (&qq)[DH / 8], float& vv, const float* __restrict__ buf, int jj,
                     int w, int row0, int c) {
    using L = FS<DH>;
    constexpr int R = L::R;
    if constexpr (R % 4 == 0) {
#pragma unroll
        for (int j = 0; j < R; j += 4) {
            const float4 a = *reinterpret_cast<const float4*>(buf + jj * DH + row0 + j);
            const float4 e = *reinterpret_cast<const float4*>(buf + L::KQ_F + jj * DH + row0 + j);
            kk[j] = a.x; kk[j + 1] = a.y; kk[j + 2] = a.z; kk[j + 3] = a.w;
            qq[j] = e.x; qq[j + 1] = e.y; qq[j + 2] = e.z; qq[j + 3] = e.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            kk[j] = buf[jj * DH + row0 + j];
            qq[j] = buf[L::KQ_F + jj * DH + row0 + j];
        }
    }
    vv = buf[2 * L::KQ_F + (w * L::CK + jj) * 8 + c];
}

// The CK steps of one chunk for this lane's slice s of its column
// (rust/src/delta.rs:289-314 per step).  Lane p of the column group returns
// the raw o and S^T k of step p in hold_o / hold_s.
//   SC = false: s is the state; S <- alpha S + k u^T (two operations per element).
//   SC = true:  s is S / G_j, G_j = alpha_0 ... alpha_{j-1} of the chunk, so the
//     update is s <- s + k (u / G_{j+1})^T, one FMA per element; with x = s^T k,
//     u / G_{j+1} = beta (v / G_{j+1} - x), and the caller scales hold_s by G_j
//     and hold_o by G_{j+1}.  rl (lane j) = 1 / G_{j+1}.
template <int DH, bool SC>
ASCA_DEV void fwd_steps(float (&s)[DH / 8], const float* __restrict__ buf, float gcur, float rl, int w, int row0,
                        int c, int p, float& hold_o, float& hold_s) {
    using L = FS<DH>;
    constexpr int R = L::R, CK = L::CK;
    static_assert(L::G == CK, "one batched store per chunk");
    float kk[2][R], qq[2][R], vv[2];
    fwd_rd<DH>(kk[0], qq[0], vv[0], buf, 0, w, row0, c);
#pragma unroll
    for (int jj = 0; jj < CK; ++jj) {
        if (jj + 1 < CK) fwd_rd<DH>(kk[(jj + 1) & 1], qq[(jj + 1) & 1], vv[(jj + 1) & 1], buf, jj + 1, w, row0, c);
        const int cs = jj & 1;
        const float bt = readlane_f(gcur, CK + jj);
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int j = 0; j < R; j += 2) {
            a0 = fmaf(s[j], kk[cs][j], a0);
            a1 = fmaf(s[j + 1], kk[cs][j + 1], a1);
        }
        const float x = group_sum<8>(a0 + a1);
        float o0 = 0.0f, o1 = 0.0f;
        if constexpr (SC) {
            const float ut = bt * fmaf(vv[cs], readlane_f(rl, jj), -x);
#pragma unroll
            for (int j = 0; j < R; j += 2) {
                s[j] = fmaf(kk[cs][j], ut, s[j]);
                s[j + 1] = fmaf(kk[cs][j + 1], ut, s[j + 1]);
                o0 = fmaf(s[j], qq[cs][j], o0);
                o1 = fmaf(s[j + 1], qq[cs][j + 1], o1);
            }
        } else {
            const float a = readlane_f(gcur, jj);
            const float u = bt * (vv[cs] - a * x);
#pragma unroll
            for (int j = 0; j < R; j += 2) {
                s[j] = a * s[j] + kk[cs][j] * u;
                s[j + 1] = a * s[j + 1] + kk[cs][j + 1] * u;
                o0 = fmaf(s[j], qq[cs][j], o0);
                o1 = fmaf(s[j + 1], qq[cs][j + 1], o1);
            }
        }
        const float oo = group_sum<8>(o0 + o1);
        hold_o = (p == jj) ? oo : hold_o;
        hold_s = (p == jj) ? x : hold_s;
    }
}

// A lane's rows row0 .. row0+R-1 of column col into a checkpoint slot (S^T,
// contiguous per column); masked elements go to the trash.
template <int R, bool EXACT>
ASCA_DEV void store_ckpt(float* __restrict__ dst, const float (&s)[R], bool col_ok, int row0, int dh,
                         float* __restrict__ tr) {
    if constexpr (EXACT && R % 4 == 0) {
#pragma unroll
        for (int j = 0; j < R; j += 4)
            *reinterpret_cast<float4*>(dst + j) = make_float4(s[j], s[j + 1], s[j + 2], s[j + 3]);
    } else {
#pragma unroll
        for (int j = 0; j < R; ++j) *((col_ok && row0 + j < dh) ? dst + j : tr + j) = s[j];
    }
}

// One block per (sequence, head) unit, unit = h*B + b (the reference's s_pre
// order, rust/src/delta.rs:54-56).  ckpt: nslots = ceil(T/CK) + 1 states per
// unit, slot j = S^T before step j*CK (element (a, i) of S at [i*dh + a]), the
// last slot S^T after step T-1.  Steps past T (the tail of the last chunk) run
// with alpha = 1, beta = 0, which leaves the state unchanged.
template <int DH, int CS, bool EXACT>
__global__ __launch_bounds__((FS<DH, CS>::NT)) void delta_fwd_k(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ alpha, const float* __restrict__ beta, float* __restrict__ o,
    float* __restrict__ sk_out, float* __restrict__ ckpt, int B, int T, int H, int dh, int nslots) {
    using L = FS<DH, CS>;
    constexpr int R = L::R, CK = L::CK;
    static_assert(2 * CK <= 16, "chunk layout: the gates of a chunk fit one 16-lane row");
    __shared__ float4 lds4[2 * L::BUF_F / 4];
    float* const lds = reinterpret_cast<float*>(lds4);

    const int unit = blockIdx.x / CS, part = blockIdx.x - unit * CS;
    const int h = unit / B, b = unit - h * B;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wg = part * L::W + w;
    const int p = lane & 7, c = lane >> 3;
    const int col = wg * 8 + c;
    const int row0 = p * R;
    const long d = (long)H * dh;
    const long dh2 = (long)dh * dh;
    const long ubase = (long)b * T * d + (long)h * dh;
    float* ob = o + ubase;
    float* skb = sk_out + ubase;
    const long gbase = (long)b * T * H + h;
    float* ckb = ckpt + (long)unit * nslots * dh2;
    const bool col_ok = EXACT || col < dh;
    float* const tr = trash_f(threadIdx.x * 2);
    const int nchunk = (T + CK - 1) / CK;

    // gates of a chunk: lane l < CK holds alpha of step t0+l, CK <= l < 2CK beta of t0+l-CK
    const int gl = lane & (2 * CK - 1);
    const float* gsrc = (gl < CK ? alpha : beta) + gbase;
    const int gstep = gl % CK;

    float s[R];
#pragma unroll
    for (int j = 0; j < R; ++j) s[j] = 0.0f;

    FwdStage<DH, CS> stg;
    fwd_stage_load<DH, CS, EXACT>(stg, 0, q, k, v, ubase, d, T, dh, wg, lane);
    // a gate of step t (lane-dependent: alpha or beta); past T, alpha = 1 and beta = 0
    const float gpad = gl < CK ? 1.0f : 0.0f;
    auto gate = [&](int t) {
        const float x = gsrc[(long)min(t, T - 1) * H];
        return t < T ? x : gpad;
    };
    float gnext = gate(gstep);
    fwd_stage_store<DH, CS>(stg, lds, w, lane);
    lds_barrier();

    for (int ci = 0; ci < nchunk; ++ci) {
        const int t0 = ci * CK;
        const float* buf = lds + (ci & 1) * L::BUF_F;
        const float gcur = gnext;
        gnext = gate(t0 + CK + gstep);
        fwd_stage_load<DH, CS, EXACT>(stg, min(ci + 1, nchunk - 1), q, k, v, ubase, d, T, dh, wg, lane);
        store_ckpt<R, EXACT>(ckb + (long)ci * dh2 + (long)col * dh + row0, s, col_ok, row0, dh, tr);
        // Lanes j < CK of gcur hold the chunk's alpha; when all of them lie in
        // [2^-8, 2^8] the chunk runs on the scaled state (fwd_steps).
        const bool bad = lane < CK && !(gcur >= 0x1p-8f && gcur <= 0x1p8f);
        float hold_o = 0.0f, hold_s = 0.0f, fo = 1.0f, fs = 1.0f;
        if (__ballot(bad) == 0) {
            // G_{j+1} = alpha_0 ... alpha_j in lane j (and in lane j of every 2CK group)
            const float pr = prefix_prod<CK>((lane & (2 * CK - 1)) < CK ? gcur : 1.0f);
            const float rl = __builtin_amdgcn_rcpf(pr);
            // both permutes run on every lane: a permute reads 0 from lanes that
            // are switched off
            fo = __shfl(pr, p & (CK - 1));
            const float fprev = __shfl(pr, (p + CK - 1) & (CK - 1));
            fs = p == 0 ? 1.0f : fprev;
            fwd_steps<DH, true>(s, buf, gcur, rl, w, row0, c, p, hold_o, hold_s);
            const float gend = readlane_f(pr, CK - 1);
#pragma unroll
            for (int j = 0; j < R; ++j) s[j] *= gend;
        } else {
            fwd_steps<DH, false>(s, buf, gcur, 0.0f, w, row0, c, p, hold_o, hold_s);
        }
        {   // lane p of the column group holds the results of step t0 + p
            const int ts = t0 + p;
            const bool ok = p < CK && ts < T && col_ok;
            *(ok ? ob + (long)ts * d + col : tr) = hold_o * fo;
            *(ok ? skb + (long)ts * d + col : tr + 1) = hold_s * fs;
        }
        fwd_stage_store<DH, CS>(stg, lds + ((ci + 1) & 1) * L::BUF_F, w, lane);
        lds_barrier();
    }
    store_ckpt<R, EXACT>(ckb + (long)nchunk * dh2 + (long)col * dh + row0, s, col_ok, row0, dh, tr);
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
        float kk[R], qq[R];
        const float* kt = k + ubase + (long)t * d;
        const float* qt = q + ubase + (long)t * d;
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const bool ok = row0 + j < dh;
            kk[j] = ok ? kt[row0 + j] : 0.0f;
            qq[j] = ok ? qt[row0 + j] : 0.0f;
        }
        const float vv = col < dh ? v[ubase + (long)t * d + col] : 0.0f;
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

// ----------------------------------------------------------------- backward
//
// Shape of the backward: a unit runs on DH/8 waves (two per SIMD at dh = 64),
// each owning 8 value columns.  Lane (rg = lane & 15, cg = lane >> 4) owns rows
// rg*M .. rg*M+M-1 (M = DH/16) of columns colb, colb+1 (colb = 8w + 2cg).  A
// C-step segment is recomputed into registers (the stash), so both phases are
// unrolled over C steps; a tail segment past T is padded with dO = 0 steps,
// which leave dS unchanged and whose outputs are dropped.

template <int DH, int CS = 1>
struct BS {
    static constexpr int W = DH / 8 / CS;
    static constexpr int NT = 64 * W;
    static constexpr int M = DH / 16;
    static constexpr int CK = DS<DH>::CK;
    // one LDS buffer (floats); two are used alternately by consecutive segments
    static constexpr int RED_F = CK * W * DH;    // dq / dk row sums per wave
    static constexpr int RAB_F = CK * W * 2;     // dalpha / dbeta per wave
    static constexpr int STQK_F = CK * DH;       // staged q (and k) rows
    static constexpr int STW_F = W * CK * 24;    // staged dO, v, sk (8 columns each) per wave
    static constexpr int STAB_F = 8 * CK + 8;    // gate table (8 floats per step), flag, sink float4
    static constexpr int RV_F = CK * DH;          // dv rows
    static constexpr int ST_OFF = 2 * RED_F + RAB_F + RV_F;   // start of the staged operands
    static constexpr int BUF_F = ST_OFF + 2 * STQK_F + STW_F + STAB_F;
    // The next segment's checkpoint tile goes through LDS (per lane, [m][thread]
    // float2), so no wait on global memory sits at a segment's start.
    static constexpr int CKS_F = NT * M * 2;
    static constexpr size_t LDS = 2 * (size_t)BUF_F * 4 + (size_t)CKS_F * 4;
    static_assert(LDS <= 160 * 1024, "backward LDS");
    // staging registers
    static constexpr int QK4 = CK * DH / 4;             // float4 per staged tensor (q or k)
    static constexpr int NQ = (2 * QK4 + NT - 1) / NT;  // staged q/k float4 per thread
    static constexpr int W4 = CK * 6;                   // per-wave float4 of dO, v, sk
    static constexpr int NW = (W4 + 63) / 64;
};

template <int DH, int CS>
struct BStage {
    float4 rq[BS<DH, CS>::NQ], rw[BS<DH, CS>::NW];
    float rab;                    // lanes j < CK: alpha of step j, CK <= j < 2CK: beta
    float rqk;                    // the same lanes: the saved q / k norms (fused backward)
    float rck[2][BS<DH, CS>::M];  // checkpoint tile: column colb+n, rows rowb..rowb+M-1
};

// wg: the wave's index among all waves of the unit (its value columns)
template <int DH, int CS, bool EXACT, bool FUSED>
ASCA_DEV void bstage_load(BStage<DH, CS>& st, int g, const float* __restrict__ q, const float* __restrict__ k,
                          const float* __restrict__ v, const float* __restrict__ d_o,
                          const float* __restrict__ skv, const float* __restrict__ alpha,
                          const float* __restrict__ beta, const float* __restrict__ qnorm,
                          const float* __restrict__ knorm, const float* __restrict__ ckb, long ubase, long gbase,
                          long d, long dh2, int T, int H, int dh, int wg, int lane, int rowb, int colb) {
    using S = BS<DH, CS>;
    constexpr int CK = S::CK, M = S::M;
    const int t0 = g * CK;
#pragma unroll
    for (int i = 0; i < S::NQ; ++i) {
        const int f0 = (int)threadIdx.x + i * S::NT;
        const int f = f0 < 2 * S::QK4 ? f0 : 0;
        const int tsr = f >= S::QK4;
        const int fl = f - tsr * S::QK4;
        const int j = fl / (DH / 4), c4 = fl % (DH / 4);
        const long t = min(t0 + j, T - 1);
        st.rq[i] = ld4m<EXACT>((tsr ? k : q) + ubase + t * d, 4 * c4, dh);
    }
#pragma unroll
    for (int i = 0; i < S::NW; ++i) {
        const int f0 = lane + 64 * i;
        const int f = f0 < S::W4 ? f0 : 0;
        const int tsr = f / (CK * 2);          // 0: dO, 1: v, 2: sk
        const int rem = f % (CK * 2);
        const int j = rem / 2, half = rem % 2;
        const long t = min(t0 + j, T - 1);
        const float* src = tsr == 0 ? d_o : (tsr == 1 ? v : skv);
        st.rw[i] = ld4m<EXACT>(src + ubase + t * d, wg * 8 + half * 4, dh);
    }
    {
        const int gl = lane & (2 * CK - 1);
        const long t = min(t0 + gl % CK, T - 1);
        st.rab = (gl < CK ? alpha : beta)[gbase + t * H];
        st.rqk = FUSED ? (gl < CK ? qnorm : knorm)[gbase + t * H] : 0.0f;
    }
    const float* cks = ckb + (long)g * dh2;
#pragma unroll
    for (int n = 0; n < 2; ++n) {
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

// Registers -> the LDS buffer of segment g (q, k rows, the waves' dO / v / sk
// columns, the gate table) and this thread's checkpoint slot cks.  Every lane
// stores, lanes without an element into the buffer's sink slot: a store that
// only some lanes make lets the compiler move the matching load down to it,
// which turns the prefetch into a wait.  Padded steps (t >= T) get dO = 0 here.
template <int DH, int CS>
ASCA_DEV void bstage_store(const BStage<DH, CS>& st, int g, int T, float* __restrict__ st_q,
                           float* __restrict__ st_k, float* __restrict__ st_w, float* __restrict__ st_ab,
                           float2* __restrict__ cks, int w, int lane) {
    using S = BS<DH, CS>;
    constexpr int CK = S::CK;
    float* const sink = st_ab + 8 * CK + 4;
#pragma unroll
    for (int m = 0; m < S::M; ++m) cks[m * S::NT] = make_float2(st.rck[0][m], st.rck[1][m]);
#pragma unroll
    for (int i = 0; i < S::NQ; ++i) {
        const int f0 = (int)threadIdx.x + i * S::NT;
        const bool ok = f0 < 2 * S::QK4;
        const int f = ok ? f0 : 0;
        const int tsr = f >= S::QK4;
        const int fl = f - tsr * S::QK4;
        const int j = fl / (DH / 4), c4 = fl % (DH / 4);
        *reinterpret_cast<float4*>(ok ? (tsr ? st_k : st_q) + j * DH + 4 * c4 : sink) = st.rq[i];
    }
#pragma unroll
    for (int i = 0; i < S::NW; ++i) {
        const int f0 = lane + 64 * i;
        const bool ok = f0 < S::W4;
        const int f = ok ? f0 : 0;
        const int tsr = f / (CK * 2);
        const int rem = f % (CK * 2);
        const int j = rem / 2, half = rem % 2;
        float4 x = st.rw[i];
        if (tsr == 0 && g * CK + j >= T) x = make_float4(0.f, 0.f, 0.f, 0.f);   // padded steps carry dO = 0
        *reinterpret_cast<float4*>(ok ? st_w + (w * CK + j) * 24 + tsr * 8 + half * 4 : sink) = x;
    }
    // Gate table, row j: alpha_j, beta_j, G_{j+1}, 1/G_{j+1}, 1/alpha_j, |q_j|,
    // |k_j| with G_{j+1} = alpha_0 ... alpha_j of the segment; st_ab[8 CK] = 1
    // when every alpha of the segment lies in [2^-8, 2^8] (the range of the
    // scaled form).  Wave 0 writes it; the other waves compute it into the sink.
    const bool w0 = w == 0;
    const bool ga = lane < CK;
    const int row = ga ? lane : lane - CK;
    const bool gl = w0 && lane < 2 * CK;
    *(gl ? st_ab + row * 8 + (ga ? 0 : 1) : sink) = st.rab;
    *(gl ? st_ab + row * 8 + (ga ? 5 : 6) : sink + 1) = st.rqk;
    const float pr = prefix_prod<CK>(ga ? st.rab : 1.0f);
    const bool wa = w0 && ga;
    *(wa ? st_ab + lane * 8 + 2 : sink) = pr;
    *(wa ? st_ab + lane * 8 + 3 : sink + 1) = __builtin_amdgcn_rcpf(pr);
    *(wa ? st_ab + lane * 8 + 4 : sink + 2) = __builtin_amdgcn_rcpf(st.rab);
    const bool bad = ga && !(st.rab >= 0x1p-8f && st.rab <= 0x1p8f);
    const bool in_range = __ballot(bad) == 0;
    *(w0 && lane == 0 ? st_ab + 8 * CK : sink + 3) = in_range ? 1.0f : 0.0f;
}

// LDS operands of reverse step j: q, k rows and the dO, v, sk column pairs.
template <int M>
struct BOps {
    float q[M], k[M];
    float2 dO, v, sk;
    float a, b, g1, r1, ia;   // gate table row of the step
};

template <int DH>
ASCA_DEV void bops_read(BOps<DH / 16>& o, const float* __restrict__ st_q, const float* __restrict__ st_k,
                        const float* __restrict__ st_w, const float* __restrict__ st_ab, int j, int w, int rowb,
                        int cg) {
    constexpr int M = DH / 16, CK = BS<DH>::CK;
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
    const float* sw = st_w + (w * CK + j) * 24 + cg * 2;
    o.dO = *reinterpret_cast<const float2*>(sw);
    o.v = *reinterpret_cast<const float2*>(sw + 8);
    o.sk = *reinterpret_cast<const float2*>(sw + 16);
    const float4 gt = *reinterpret_cast<const float4*>(st_ab + 8 * j);
    o.a = gt.x;
    o.b = gt.y;
    o.g1 = gt.z;
    o.r1 = gt.w;
    o.ia = st_ab[8 * j + 4];
}

// One reverse step of the BPTT for this lane's tile (rust/src/delta.rs:485-572
// reorganised per value column).  sm / sa: tiles of S before / after the step
// from the register stash.  Updates ds in place, stores dv, and leaves the dq /
// dk row sums and the dalpha / dbeta totals of this wave in LDS for the epilogue.
//   SC = false: ds is dS, sm / sa are S.
//   SC = true: with G_j = alpha_0 ... alpha_{j-1} of the segment, ds holds
//     G_{j+1} dS, sm = S_before / G_j and sa = S_after / G_{j+1}; then
//     dS <- alpha dS + k dsk^T becomes ds <- ds + k (-beta du~)^T with
//     du~ = ds^T k = G_{j+1} du (one FMA per element), and every output term
//     takes its scale from the step's gate-table row (g1 = G_{j+1}, r1 = 1/G_{j+1},
//     ia = 1/alpha = G_j / G_{j+1}).
template <int DH, bool EXACT, bool SC>
ASCA_DEV void bwd_step(const BOps<DH / 16>& in, const float (&sm)[DH / 16][2], const float (&sa)[DH / 16][2],
                       float (&ds)[DH / 16][2], float* __restrict__ rq, float* __restrict__ rk, float& pab_out,
                       float* __restrict__ rv, int rg, int cg,
                       int rowb, int colb, int dh) {
    constexpr int M = DH / 16;
    const float a = in.a, bb = in.b;
    const float vv[2] = {in.v.x, in.v.y};
    const float sk[2] = {in.sk.x, in.sk.y};
    float dO[2] = {in.dO.x, in.dO.y};
    if constexpr (SC) {
        dO[0] *= in.g1;
        dO[1] *= in.g1;
    }

    // dS += q dO^T  (delta.rs:508-511)
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int n = 0; n < 2; ++n) ds[m][n] = fmaf(in.q[m], dO[n], ds[m][n]);
    // du = dS^T k  (delta.rs:536-542): 16-lane butterfly over row groups
    float dut[2];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        float acc = 0.0f;
#pragma unroll
        for (int m = 0; m < M; ++m) acc = fmaf(ds[m][n], in.k[m], acc);
        dut[n] = group_sum<16>(acc);
    }
    // du: true du; uh: the u that multiplies ds; sh: the dsk that multiplies sm
    // and updates ds
    float du[2], wv[2], uh[2], sh[2];
    const float cu = SC ? bb * in.r1 : bb;
    const float cs = SC ? -bb : -bb * a;
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        du[n] = SC ? dut[n] * in.r1 : dut[n];
        wv[n] = vv[n] - a * sk[n];
        uh[n] = cu * wv[n];
        sh[n] = cs * dut[n];
    }
    // dv = beta du  (delta.rs:550): the lanes of row group 0 put it in the
    // step's LDS row; the epilogue stores whole rows
    if (rg == 0) *reinterpret_cast<float2*>(rv + colb) = make_float2(bb * du[0], bb * du[1]);

    // Off-critical-path partial sums over this lane's 2 columns.
    //   dq = S_t dO                                       (delta.rs:504-507)
    //   dk = dS u + S_{t-1} dsk                           (delta.rs:532-534, 556-558)
    //   dalpha = <dS, S_{t-1}> - beta du.sk               (delta.rs:530, 552)
    //   dbeta = du.(v - alpha sk)                         (delta.rs:549)
    float pq[M], pk[M];
    float pa0 = 0.0f, pa1 = 0.0f;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        pq[m] = fmaf(sa[m][1], dO[1], sa[m][0] * dO[0]);
        float xk = uh[0] * ds[m][0];
        xk = fmaf(uh[1], ds[m][1], xk);
        xk = fmaf(sh[0], sm[m][0], xk);
        pk[m] = fmaf(sh[1], sm[m][1], xk);
        pa0 = fmaf(ds[m][0], sm[m][0], pa0);
        pa1 = fmaf(ds[m][1], sm[m][1], pa1);
    }
    const float ea = fmaf(-bb * du[1], sk[1], -bb * du[0] * sk[0]);
    const float eb = fmaf(du[1], wv[1], du[0] * wv[0]);
    const float pab = SC ? (pa0 + pa1) * in.ia : pa0 + pa1;
    float pa = pab + (rg == 0 ? ea : 0.0f);
    float pb = rg == 0 ? eb : 0.0f;

    // dS <- alpha dS + k dsk^T  (delta.rs:543-545, 559-563)
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int n = 0; n < 2; ++n) ds[m][n] = SC ? fmaf(in.k[m], sh[n], ds[m][n]) : a * ds[m][n] + in.k[m] * sh[n];

    // Column sums of pq, pk over the 4 column groups (lane bits 4,5),
    // transposed so each lane keeps whole-row sums.
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
    // first level of the cross-step reduction of (dalpha, dbeta): lanes < 32
    // keep the dalpha pair sum, lanes >= 32 the dbeta one
    pab_out = tsum32(pa, pb);
}

// One segment of CK steps (t0 .. t0+CK-1): recompute the states from the
// checkpoint s0 into the register stash (phase A), then run the steps in
// reverse (phase B), storing the next segment's staged operands (stg) into its
// LDS buffer nbuf halfway, and reduce the per-step dalpha / dbeta partials.  With SC
// the stash holds S / G_j and ds is carried as G_{j+1} dS inside the segment
// (see bwd_step); ds enters and leaves unscaled.
template <int DH, int CS, bool EXACT, bool SC>
ASCA_DEV void bwd_segment(const float (&s0)[DH / 16][2], float (&ds)[DH / 16][2], const BStage<DH, CS>& stg,
                          float* __restrict__ nbuf, float2* __restrict__ cks, const float* __restrict__ st_q,
                          const float* __restrict__ st_k, const float* __restrict__ st_w,
                          const float* __restrict__ st_ab, float* __restrict__ red_q, float* __restrict__ red_k,
                          float* __restrict__ red_ab, float* __restrict__ red_v, int t0,
                          int T, int w, int lane, int rg, int cg, int rowb, int colb, int dh) {
    using S = BS<DH, CS>;
    constexpr int M = S::M, CK = S::CK, W = S::W;
    // stash[j] = S before step t0 + j, stash[CK] = S after the segment's last step
    float stash[CK + 1][M][2];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        stash[0][m][0] = s0[m][0];
        stash[0][m][1] = s0[m][1];
    }
    // ---- phase A: S_{t0+1} .. S_{t0+CK}
#pragma unroll
    for (int j = 1; j <= CK; ++j) {
        const int jp = j - 1;
        float km[M];
#pragma unroll
        for (int m = 0; m < M; ++m) km[m] = st_k[jp * DH + rowb + m];
        const float* sw = st_w + (w * CK + jp) * 24 + cg * 2;
        const float2 vv = *reinterpret_cast<const float2*>(sw + 8);
        const float2 sk = *reinterpret_cast<const float2*>(sw + 16);
        const float4 gt = *reinterpret_cast<const float4*>(st_ab + 8 * jp);
        const float a = gt.x, bt = gt.y;
        float u0 = bt * (vv.x - a * sk.x), u1 = bt * (vv.y - a * sk.y);
        if constexpr (SC) {
            u0 *= gt.w;
            u1 *= gt.w;
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            if constexpr (SC) {
                stash[j][m][0] = fmaf(km[m], u0, stash[jp][m][0]);
                stash[j][m][1] = fmaf(km[m], u1, stash[jp][m][1]);
            } else {
                stash[j][m][0] = a * stash[jp][m][0] + km[m] * u0;
                stash[j][m][1] = a * stash[jp][m][1] + km[m] * u1;
            }
        }
    }
    if constexpr (SC) {
        const float gend = st_ab[8 * (CK - 1) + 2];
#pragma unroll
        for (int m = 0; m < M; ++m) {
            ds[m][0] *= gend;
            ds[m][1] *= gend;
        }
    }

    // ---- phase B: steps t0+CK-1 .. t0 in reverse, LDS operands one step ahead
    BOps<M> op[2];
    float pab[CK];
    bops_read<DH>(op[(CK - 1) & 1], st_q, st_k, st_w, st_ab, CK - 1, w, rowb, cg);
#pragma unroll
    for (int jj = CK - 1; jj >= 0; --jj) {
        if (jj > 0) bops_read<DH>(op[(jj - 1) & 1], st_q, st_k, st_w, st_ab, jj - 1, w, rowb, cg);
        bwd_step<DH, EXACT, SC>(op[jj & 1], stash[jj], stash[jj + 1], ds, red_q + (jj * W + w) * DH,
                                red_k + (jj * W + w) * DH, pab[jj], red_v + jj * DH, rg, cg, rowb, colb, dh);
        if (jj == CK / 2) {
            // the staged operands of the next segment (loads issued at the
            // segment's start) go to its buffer; the fence keeps the scheduler
            // from hoisting the stores, and their wait, to the segment's start
            __builtin_amdgcn_sched_barrier(0);
            float* const n_q = nbuf + S::ST_OFF;
            float* const n_k = n_q + S::STQK_F;
            float* const n_w = n_k + S::STQK_F;
            bstage_store<DH, CS>(stg, t0 > 0 ? t0 / CK - 1 : 0, T, n_q, n_k, n_w, n_w + S::STW_F, cks, w, lane);
        }
    }
    cross_step_sum<CK, W>(pab, red_ab, w, lane);
}

// Backward of one unit per block (CS = 1), or of half of its value columns
// per block (CS = 2).  Output pointers are already offset to the head-0 column
// of their quantity; element (r, h*dh + i) is at ptr[r*ldx + h*dh + i] and the
// per-head scalars at ga[r*ldg + h].  FUSED applies the L2-norm backward
// (rust/src/delta.rs:677-698) and the sigmoid backward (delta.rs:602-611).
// With CS = 2 the row sums dq, dk and dalpha, dbeta cover only the block's
// columns: they go to the partial buffers (part_x [CS][B*T][H*dh], part_g
// [CS][B*T][2H]) and delta_combine_k finishes them; dv is complete per column.
template <int DH, int CS, bool EXACT, bool FUSED>
__global__ __launch_bounds__((BS<DH, CS>::NT)) void delta_bwd_k(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ alpha, const float* __restrict__ beta, const float* __restrict__ d_o,
    const float* __restrict__ skv, const float* __restrict__ ckpt, const float* __restrict__ qnorm,
    const float* __restrict__ knorm, float* __restrict__ gq, float* __restrict__ gk,
    float* __restrict__ gv, long ldx, float* __restrict__ ga, float* __restrict__ gb, long ldg,
    float* __restrict__ part_x, float* __restrict__ part_g, int B, int T, int H, int dh, int nslots) {
    using S = BS<DH, CS>;
    constexpr int M = S::M, W = S::W, CK = S::CK;
    extern __shared__ float4 lds4[];
    float* const lds = reinterpret_cast<float*>(lds4);
    float2* const cks = reinterpret_cast<float2*>(lds4 + 2 * S::BUF_F / 4) + threadIdx.x;   // checkpoint slot

    const int unit = blockIdx.x / CS, part = blockIdx.x - unit * CS;
    const int h = unit / B, b = unit - h * B;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wg = part * W + w;
    const int rg = lane & 15, cg = lane >> 4;
    const int colb = wg * 8 + cg * 2;
    const int rowb = rg * M;
    const long d = (long)H * dh;
    const long dh2 = (long)dh * dh;
    const long ubase = (long)b * T * d + (long)h * dh;
    const long gbase = (long)b * T * H + h;
    const long hoff = (long)h * dh;
    const float* ckb = ckpt + (long)unit * nslots * dh2;
    const int nseg = (T + CK - 1) / CK;

    float ds[M][2];
#pragma unroll
    for (int m = 0; m < M; ++m) ds[m][0] = ds[m][1] = 0.0f;

    BStage<DH, CS> stg;
    bstage_load<DH, CS, EXACT, FUSED>(stg, nseg - 1, q, k, v, d_o, skv, alpha, beta, qnorm, knorm, ckb, ubase,
                                      gbase, d, dh2, T, H, dh, wg, lane, rowb, colb);
    {
        float* const b0 = lds + ((nseg - 1) & 1) * S::BUF_F + S::ST_OFF;
        bstage_store<DH, CS>(stg, nseg - 1, T, b0, b0 + S::STQK_F, b0 + 2 * S::STQK_F,
                             b0 + 2 * S::STQK_F + S::STW_F, cks, w, lane);
    }
    for (int g = nseg - 1; g >= 0; --g) {
        const int t0 = g * CK;
        float* const buf = lds + (g & 1) * S::BUF_F;
        float* const nbuf = lds + ((g + 1) & 1) * S::BUF_F;   // the next segment's (g - 1)
        float* const red_q = buf;                        // [CK][W][DH]
        float* const red_k = red_q + S::RED_F;           // [CK][W][DH]
        float* const red_ab = red_k + S::RED_F;          // [CK][W][2]
        float* const red_v = red_ab + S::RAB_F;          // [CK][DH]
        float* const st_q = buf + S::ST_OFF;             // [CK][DH]
        float* const st_k = st_q + S::STQK_F;            // [CK][DH]
        float* const st_w = st_k + S::STQK_F;            // [W][CK][24]
        float* const st_ab = st_w + S::STW_F;            // [CK][8] gate table + flag

        float s0[M][2];   // checkpoint: S before step t0 (this thread's slot)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float2 x = cks[m * S::NT];
            s0[m][0] = x.x;
            s0[m][1] = x.y;
        }
        bstage_load<DH, CS, EXACT, FUSED>(stg, g > 0 ? g - 1 : 0, q, k, v, d_o, skv, alpha, beta, qnorm, knorm, ckb,
                                          ubase, gbase, d, dh2, T, H, dh, wg, lane, rowb, colb);
        lds_barrier();  // staging of this segment visible to all waves

        if (__builtin_amdgcn_readfirstlane(__float_as_int(st_ab[8 * CK])) == __float_as_int(1.0f))
            bwd_segment<DH, CS, EXACT, true>(s0, ds, stg, nbuf, cks, st_q, st_k, st_w, st_ab, red_q, red_k,
                                             red_ab, red_v, t0, T, w, lane, rg, cg, rowb, colb, dh);
        else
            bwd_segment<DH, CS, EXACT, false>(s0, ds, stg, nbuf, cks, st_q, st_k, st_w, st_ab, red_q, red_k,
                                              red_ab, red_v, t0, T, w, lane, rg, cg, rowb, colb, dh);
        lds_barrier();  // red_* of this segment complete

        // ---- phase C: cross-wave sums, optional norm/sigmoid backward, stores
        constexpr int NA = (DH + 63) / 64;
        for (int jj = w; jj < CK && t0 + jj < T; jj += W) {
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
                    dq[ia] = red_q[jj * W * DH + a];
                    dk[ia] = red_k[jj * W * DH + a];
#pragma unroll
                    for (int w2 = 1; w2 < W; ++w2) {
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
            float dA, dB;
            {
                const float2 x = *reinterpret_cast<const float2*>(red_ab + jj * W * 2);
                dA = x.x;
                dB = x.y;
            }
#pragma unroll
            for (int w2 = 1; w2 < W; ++w2) {
                const float2 x = *reinterpret_cast<const float2*>(red_ab + (jj * W + w2) * 2);
                dA += x.x;
                dB += x.y;
            }
            // dv: complete per column; this block's columns are [part DH/CS, (part+1) DH/CS)
#pragma unroll
            for (int ia = 0; ia < NA; ++ia) {
                const int a = lane + 64 * ia;
                if (a < DH / CS && part * (DH / CS) + a < dh)
                    gv[r * ldx + hoff + part * (DH / CS) + a] = red_v[jj * DH + part * (DH / CS) + a];
            }
            if constexpr (CS > 1) {
                float* const px = part_x + ((long)part * B * T + r) * d + hoff;
#pragma unroll
                for (int ia = 0; ia < NA; ++ia) {
                    const int a = lane + 64 * ia;
                    if (a < dh) {
                        px[a] = dq[ia];
                        px[(long)B * T * d * CS + a] = dk[ia];
                    }
                }
                if (lane == 0) {
                    float* const pg = part_g + ((long)part * B * T + r) * 2 * H;
                    pg[h] = dA;
                    pg[H + h] = dB;
                }
            } else if constexpr (FUSED) {
                dotq = wave_sum(dotq);
                dotk = wave_sum(dotk);
                // 1/|q|, 1/|k| by the hardware reciprocal (within 1 ulp)
                const float iqn = __builtin_amdgcn_rcpf(st_ab[8 * jj + 5]);
                const float ikn = __builtin_amdgcn_rcpf(st_ab[8 * jj + 6]);
#pragma unroll
                for (int ia = 0; ia < NA; ++ia) {
                    const int a = lane + 64 * ia;
                    if (a < dh) {
                        gq[r * ldx + hoff + a] = (dq[ia] - qa[ia] * dotq) * iqn;
                        gk[r * ldx + hoff + a] = (dk[ia] - ka[ia] * dotk) * ikn;
                    }
                }
                if (lane == 0) {
                    const float al = st_ab[8 * jj], be = st_ab[8 * jj + 1];
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

// Finish a column-split backward: sum the CS = 2 partial row sums of dq, dk
// and dalpha, dbeta and apply the fused norm / sigmoid backward as
// delta_bwd_k does for CS = 1.  One wave per (row, head).
template <bool FUSED>
__global__ __launch_bounds__(256) void delta_combine_k(
    const float* __restrict__ part_x, const float* __restrict__ part_g, const float* __restrict__ q,
    const float* __restrict__ k, const float* __restrict__ alpha, const float* __restrict__ beta,
    const float* __restrict__ qnorm, const float* __restrict__ knorm, float* __restrict__ gq,
    float* __restrict__ gk, long ldx, float* __restrict__ ga, float* __restrict__ gb, long ldg, long rows, int H,
    int dh) {
    const long id = (long)blockIdx.x * 4 + (threadIdx.x >> 6);  // r * H + h
    if (id >= rows * H) return;
    const int lane = threadIdx.x & 63;
    const long r = id / H;
    const int h = (int)(id - r * H);
    const long d = (long)H * dh, n = rows * d;
    const long o = r * d + (long)h * dh;
    // every load issued first (indices clamped into the head, lanes past dh
    // masked afterwards): a load under a per-lane condition is waited for on
    // its own
    float x0[2], x1[2], x2[2], x3[2], qa[2], ka[2];
#pragma unroll
    for (int ia = 0; ia < 2; ++ia) {
        const long a = o + min(lane + 64 * ia, dh - 1);
        x0[ia] = part_x[a];
        x1[ia] = part_x[n + a];
        x2[ia] = part_x[2 * n + a];
        x3[ia] = part_x[3 * n + a];
        if constexpr (FUSED) {
            qa[ia] = q[a];
            ka[ia] = k[a];
        }
    }
    const long og = r * 2 * H + h, ng = rows * 2 * H;
    const float g0 = part_g[og], g1 = part_g[ng + og], g2 = part_g[og + H], g3 = part_g[ng + og + H];
    float qn = 1.0f, kn = 1.0f, al = 0.0f, be = 0.0f;
    if constexpr (FUSED) {
        qn = qnorm[r * H + h];
        kn = knorm[r * H + h];
        al = alpha[r * H + h];
        be = beta[r * H + h];
    }
    float dq[2], dk[2];
    float dotq = 0.0f, dotk = 0.0f;
#pragma unroll
    for (int ia = 0; ia < 2; ++ia) {
        const bool ok = lane + 64 * ia < dh;
        dq[ia] = ok ? x0[ia] + x1[ia] : 0.0f;
        dk[ia] = ok ? x2[ia] + x3[ia] : 0.0f;
        if constexpr (FUSED) {
            qa[ia] = ok ? qa[ia] : 0.0f;
            ka[ia] = ok ? ka[ia] : 0.0f;
            dotq = fmaf(qa[ia], dq[ia], dotq);
            dotk = fmaf(ka[ia], dk[ia], dotk);
        }
    }
    const float dA = g0 + g1;
    const float dB = g2 + g3;
    if constexpr (FUSED) {
        dotq = wave_sum(dotq);
        dotk = wave_sum(dotk);
#pragma unroll
        for (int ia = 0; ia < 2; ++ia) {
            const int a = lane + 64 * ia;
            if (a < dh) {
                gq[r * ldx + (long)h * dh + a] = (dq[ia] - qa[ia] * dotq) / qn;
                gk[r * ldx + (long)h * dh + a] = (dk[ia] - ka[ia] * dotk) / kn;
            }
        }
        if (lane == 0) {
            ga[r * ldg + h] = dA * al * (1.0f - al);
            gb[r * ldg + h] = dB * be * (1.0f - be);
        }
    } else {
#pragma unroll
        for (int ia = 0; ia < 2; ++ia) {
            const int a = lane + 64 * ia;
            if (a < dh) {
                gq[r * ldx + (long)h * dh + a] = dq[ia];
                gk[r * ldx + (long)h * dh + a] = dk[ia];
            }
        }
        if (lane == 0) {
            ga[r * ldg + h] = dA;
            gb[r * ldg + h] = dB;
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


// Units (sequence, head) at or below which each unit's value columns run on two
// blocks: half of MI355X's 256 CUs, so that a small batch still fills the chip.
// dh = 128 always splits: one block of 16 waves would cap the backward at 128
// VGPRs (1024 threads per block) and spill about 140 of them, where two
// blocks of 8 waves hold their ~215 without spilling.  A function of the shape
// only, so the workspace size never depends on the device state.
constexpr long SPLIT_UNITS = 128;
// dh = 64 always runs a block per unit on the blocked kernels of delta_ut64.hip:
// the unit's state lives in the accumulator tiles of one block's four chain
// waves.  Even the per-step dh = 64 kernels they replaced were faster on one
// block per unit than on two at any unit count (T = 1024, 8-128 units: forward
// ~150 against ~157 us, backward ~345 against ~470 us).
static int col_split(int B, int H, int dh, int dhc) {
    if (dh == 64) return 1;
    return (long)B * H <= SPLIT_UNITS || dhc == 128 ? 2 : 1;
}

static bool blocked64(int dh, int cs) { return dh == 64 && cs == 1; }

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static DeltaWs ws_layout(int B, int T, int H, int dh, void* base) {
    DeltaWs w;
    const int dhc = dh_class(dh);
    w.cs = col_split(B, H, dh, dhc);
    w.ck = blocked64(dh, w.cs) ? D64_CK : ck_for(dhc);
    w.nslots = (T + w.ck - 1) / w.ck + 1;   // the state before every chunk, then the final state
    // the blocked form keeps the u rows per unit and 16-step block (ut64_kernels.h, U_TILE)
    const size_t sk_rows = blocked64(dh, w.cs) ? (size_t)(T + D64_BLK - 1) / D64_BLK * D64_BLK : (size_t)T;
    const size_t sk_bytes = align256((size_t)B * sk_rows * H * dh * sizeof(float));
    const size_t ck_bytes = align256((size_t)B * H * w.nslots * dh * dh * sizeof(float));
    const size_t rec_bytes =
        blocked64(dh, w.cs) ? align256((size_t)B * H * ((T + D64_BLK - 1) / D64_BLK) * D64_REC * sizeof(float)) : 0;
    char* c = reinterpret_cast<char*>(base);
    w.sk = reinterpret_cast<float*>(base);
    w.ckpt = base ? reinterpret_cast<float*>(c + sk_bytes) : nullptr;
    w.rec = base && rec_bytes ? reinterpret_cast<float*>(c + sk_bytes + ck_bytes) : nullptr;
    w.bytes = sk_bytes + ck_bytes + rec_bytes;
    return w;
}

// Floats of the column-split backward's partial dq, dk and dalpha, dbeta
// (stream-ordered scratch of the backward call, never the forward's workspace).
static size_t part_floats(int cs, int B, int T, int H, int dh) {
    if (cs <= 1) return 0;
    return (size_t)2 * cs * B * T * H * dh + (size_t)cs * B * T * 2 * H;
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
    if (DH == 128 || ws.cs > 1)
        hipLaunchKernelGGL((delta_fwd_k<DH, 2, EXACT>), dim3(B * H * 2), dim3(FS<DH, 2>::NT), 0, st, q, k, v, alpha,
                           beta, o, ws.sk, ws.ckpt, B, T, H, dh, ws.nslots);
    else if constexpr (DH < 128)  // dh = 128 always splits its columns
        hipLaunchKernelGGL((delta_fwd_k<DH, 1, EXACT>), dim3(B * H), dim3(FS<DH, 1>::NT), 0, st, q, k, v, alpha,
                           beta, o, ws.sk, ws.ckpt, B, T, H, dh, ws.nslots);
    return post_launch("delta_fwd");
}

static int launch_fwd(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                      float* o, const DeltaWs& ws, int B, int T, int H, int dh, hipStream_t st) {
    const int dhc = dh_class(dh);
    const bool exact = dh == dhc && aligned16(q) && aligned16(k);
    if (blocked64(dh, ws.cs)) return launch_ut_fwd64(q, k, v, alpha, beta, o, ws, B, T, H, st);
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

template <int DH, int CS, bool EXACT, bool FUSED>
static int launch_bwd_cs(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                         const float* d_o, const DeltaWs& ws, const float* qn, const float* kn, float* gq, float* gk,
                         float* gv, long ldx, float* ga, float* gb, long ldg, int B, int T, int H, int dh,
                         hipStream_t st) {
    const size_t lds = BS<DH, CS>::LDS;
    if (int arc = allow_lds(reinterpret_cast<const void*>(&delta_bwd_k<DH, CS, EXACT, FUSED>), lds)) return arc;
    int rc = pre_launch("delta_bwd");
    if (rc) return rc;
    // the column halves' partials: scratch of this call on its stream
    StreamScratch sc;
    if ((rc = sc.get(part_floats(CS, B, T, H, dh), st))) return rc;
    float* part_x = sc.ws.p;
    float* part_g = CS > 1 ? part_x + (size_t)2 * CS * B * T * H * dh : nullptr;
    hipLaunchKernelGGL((delta_bwd_k<DH, CS, EXACT, FUSED>), dim3(B * H * CS), dim3(BS<DH, CS>::NT), lds, st, q, k,
                       v, alpha, beta, d_o, ws.sk, ws.ckpt, qn, kn, gq, gk, gv, ldx, ga, gb, ldg, part_x, part_g, B,
                       T, H, dh, ws.nslots);
    if ((rc = post_launch("delta_bwd"))) {
        (void)sc.release(st);
        return rc;
    }
    if (CS == 1) return sc.release(st);
    if ((rc = pre_launch("delta_combine"))) {
        (void)sc.release(st);
        return rc;
    }
    const long rows = (long)B * T;
    hipLaunchKernelGGL((delta_combine_k<FUSED>), dim3((unsigned)((rows * H + 3) / 4)), dim3(256), 0, st, part_x,
                       part_g, q, k, alpha, beta, qn, kn, gq, gk, ldx, ga, gb, ldg, rows, H, dh);
    rc = post_launch("delta_combine");
    const int rr = sc.release(st);
    return rc ? rc : rr;
}

template <int DH, bool EXACT, bool FUSED>
static int launch_bwd_t(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                        const float* d_o, const DeltaWs& ws, const float* qn, const float* kn, float* gq, float* gk,
                        float* gv, long ldx, float* ga, float* gb, long ldg, int B, int T, int H, int dh,
                        hipStream_t st) {
    if (DH == 128 || ws.cs > 1)
        return launch_bwd_cs<DH, 2, EXACT, FUSED>(q, k, v, alpha, beta, d_o, ws, qn, kn, gq, gk, gv, ldx, ga, gb, ldg,
                                                  B, T, H, dh, st);
    if constexpr (DH == 128) return fail(ASCA_ERR_UNSUPPORTED, "dh=128 without column split");
    else return launch_bwd_cs<DH, 1, EXACT, FUSED>(q, k, v, alpha, beta, d_o, ws, qn, kn, gq, gk, gv, ldx, ga, gb, ldg, B,
                                              T, H, dh, st);
}

template <bool FUSED>
static int launch_bwd(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                      const float* d_o, const DeltaWs& ws, const float* qn, const float* kn, float* gq, float* gk,
                      float* gv, long ldx, float* ga, float* gb, long ldg, int B, int T, int H, int dh,
                      hipStream_t st) {
    const int dhc = dh_class(dh);
    const bool exact = dh == dhc && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(d_o) &&
                       aligned16(gv) && ((ldx * 4) % 16 == 0);
    if (blocked64(dh, ws.cs))
        return launch_ut_bwd64(FUSED, q, k, v, alpha, beta, d_o, ws, qn, kn, gq, gk, gv, ldx, ga, gb, ldg, B, T, H, st);
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
