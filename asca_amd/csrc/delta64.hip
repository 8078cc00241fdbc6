// Gated delta rule, recurrent form, f32, dh = 64, on four waves per
// (sequence, head) unit: one wave per SIMD, 16 state elements per lane.
//
// Same math, outputs and workspace as delta.hip (DeltaBlock::scan_cpu,
// rust/src/delta.rs:244-334, and bptt_cpu, :421-613).  When every unit has a
// CU of its own (B*H > 128 on the 256 CUs of an MI355X), a unit's 4096 state
// elements fill the CU's four SIMDs with one wave each, and a lane holding 16
// elements instead of 8 halves the per-element share of all the work that is
// not a state FMA: reductions, gate scalars, operand reads.
//
//  * Forward: lane = 4c + p holds rows 16p..16p+15 of value column 16w + c, so
//    S^T k and S^T q are two-level quad DPP sums.  Each wave builds the gate
//    table of the next chunk (beta, 1/G, G) into LDS while the current chunk
//    runs, and a step reads its row as one broadcast vector (no v_readlane).
//    The k and q rows sit in LDS with row quarter p at float 20p, so the four
//    distinct 16-byte addresses of a 16-lane read fall on four distinct bank
//    groups.
//  * Backward: lane (rg = lane & 7, cg = lane >> 3) holds rows 8rg..8rg+7 of
//    columns 16w + 2cg, +1.  du = dS^T k is an 8-lane DPP sum; the column sums
//    of dq and dk are transposed swap reductions (permlane32, permlane16, one DPP
//    level) that leave every lane one whole row, written to LDS once per step.
//    There is no register stash of recomputed states.  In a segment whose gates
//    all lie in [2^-8, 2^8] the state is carried scaled, s_j = S_j / G_{j+1} with
//    G_{j+1} = alpha_0 ... alpha_j of the segment, and that scaled state changes
//    additively (s_j = s_{j-1} + k_j u~_j^T), so the walk starts from the state
//    after the segment (the next checkpoint) and steps back with
//    s_{j-1} = s_j - k_j u~_j^T: one FMA per element and step, no division by a
//    gate.  A segment outside that range (zero, tiny or huge gates) recomputes
//    every state it needs from the segment's first checkpoint instead.
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

// ================================================================== forward

constexpr int FR = 16;                       // rows per lane
constexpr int FROW = 80;                     // padded k / q row: row quarter p at float 20p
ASCA_DEV int fpad(int a) { return a + 4 * (a >> 4); }
// Chunk buffer (floats): k rows [CK][FROW], q rows [CK][FROW], v rows [CK][DH],
// one gate table per wave [W][CK][8], and a sink for the writes of lanes
// without a table row.
constexpr int F_K = 0;
constexpr int F_Q = CK * FROW;
constexpr int F_V = 2 * CK * FROW;
constexpr int F_G = F_V + DH * CK;
constexpr int F_SINK = F_G + W * CK * 8;
constexpr int F_BUF = F_SINK + 8;
static_assert(F_BUF % 4 == 0, "float4 buffers");

struct FStage {
    float4 kq[2]; // two float4 of the chunk's k or q rows
    float4 v;     // one float4 of the chunk's v rows
    float a, b;   // lane j (mod CK): alpha, beta of step t0 + j (1 and 0 past T)
};

// Global -> registers for chunk c; every lane loads (clamped addresses), so no
// load sits under a lane condition.
template <bool AL>
ASCA_DEV void fstage_load(FStage& st, int c, const float* __restrict__ q, const float* __restrict__ k,
                          const float* __restrict__ v, const float* __restrict__ alpha,
                          const float* __restrict__ beta, long ubase, long gbase, long d, int T, int H,
                          int lane) {
    const int t0 = c * CK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int f = threadIdx.x + NT * i;
        const int tsr = f >> 8, j = (f >> 4) & (CK - 1), c4 = f & 15;
        const long t = min(t0 + j, T - 1);
        st.kq[i] = ld4<AL>((tsr ? q : k) + ubase + t * d + 4 * c4);
    }
    {
        const int f = threadIdx.x;
        const int j = f >> 4, c4 = f & 15;
        const long t = min(t0 + j, T - 1);
        st.v = ld4<AL>(v + ubase + t * d + 4 * c4);
    }
    {
        const int t = t0 + (lane & (CK - 1));
        const long tc = min(t, T - 1);
        const float a = alpha[gbase + tc * H];
        const float b = beta[gbase + tc * H];
        // steps past T: alpha = 1, beta = 0 leave the state unchanged
        st.a = t < T ? a : 1.0f;
        st.b = t < T ? b : 0.0f;
    }
}

// Registers -> the chunk buffer; builds this wave's gate table, row j =
// {beta_j, 1/G_{j+1}, alpha_j, 0, G_{j+1}, G_j, 0, 0}.  Returns whether every
// alpha of the chunk lies in [2^-6, 2^6] (wave-uniform), the range in which the
// scaled state of a 16-step chunk stays within 2^+-96 of the true one.
ASCA_DEV bool fstage_store(const FStage& st, float* __restrict__ buf, int w, int lane) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int f = threadIdx.x + NT * i;
        const int tsr = f >> 8, j = (f >> 4) & (CK - 1), c4 = f & 15;
        *reinterpret_cast<float4*>(buf + (tsr ? F_Q : F_K) + j * FROW + fpad(4 * c4)) = st.kq[i];
    }
    {
        const int f = threadIdx.x;
        const int j = f >> 4, c4 = f & 15;
        *reinterpret_cast<float4*>(buf + F_V + j * DH + 4 * c4) = st.v;
    }
    const bool gl = lane < CK;
    const float pr = prefix_prod<CK>(gl ? st.a : 1.0f);   // G_{j+1} in lane j
    const float pv = dpp_or<0x111>(1.0f, pr);              // G_j (row_shr 1; lane 0 keeps 1)
    float* const row = gl ? buf + F_G + (w * CK + lane) * 8 : buf + F_SINK;
    *reinterpret_cast<float4*>(row) = make_float4(st.b, __builtin_amdgcn_rcpf(pr), st.a, 0.0f);
    *reinterpret_cast<float2*>(row + 4) = make_float2(pr, pv);
    const bool bad = gl && !(st.a >= 0x1p-6f && st.a <= 0x1p6f);
    return __ballot(bad) == 0;
}

ASCA_DEV void rd16(float (&x)[FR], const float* __restrict__ p) {
#pragma unroll
    for (int e = 0; e < FR; e += 4) {
        const float4 y = *reinterpret_cast<const float4*>(p + fpad(e));
        x[e] = y.x; x[e + 1] = y.y; x[e + 2] = y.z; x[e + 3] = y.w;
    }
}

// The CK steps of a chunk for this lane's 16 rows (rust/src/delta.rs:289-314
// per step), with the chunk's global stores spread over its steps: at the
// checkpoint-wide rate of every wave a chunk's stores issued at once queue the
// next chunk's loads behind them.  Steps 0..3 each store a quarter of the
// checkpoint ck (the state before the chunk, as S^T) to ckdst; lane p of a
// column's quad keeps the o and S^T k of step p + 4h and stores them after
// step 4h + 3 (rows past nvalid go to the trash), except the last group's,
// which it returns in last_o / last_sk (already rescaled) for the caller to
// store once the next chunk's loads are queued: loads and stores complete in
// order, and a load queued behind a fresh store waits for it.
//   SC = false: s is the state; S <- alpha S + k u^T.
//   SC = true:  s = S / G_j; x = s^T k, u / G_{j+1} = beta (v / G_{j+1} - x) and
//     s <- s + k (u / G_{j+1})^T (one FMA per element); o and S^T k are
//     rescaled by G_{j+1} and G_j at their store.
template <bool SC>
ASCA_DEV void fsteps(float (&s)[FR], const float* __restrict__ buf, const float* __restrict__ gt,
                     const float (&vv)[CK], int p, const float (&ck)[FR], float* __restrict__ ckdst,
                     float* __restrict__ od, float* __restrict__ skd, long d, int nvalid, float* __restrict__ tr,
                     float& last_o, float& last_sk) {
    const float* const kr = buf + F_K + fpad(16 * p);
    const float* const qr = buf + F_Q + fpad(16 * p);
    float kk[2][FR], qq[2][FR];
    float4 gg[2];
    float2 gs = make_float2(1.0f, 1.0f);   // G_{jj+1}, G_jj of this lane's step jj = p + 4h
    float ho = 0.0f, hs = 0.0f;
    rd16(kk[0], kr);
    rd16(qq[0], qr);
    gg[0] = *reinterpret_cast<const float4*>(gt);
#pragma unroll
    for (int j = 0; j < CK; ++j) {
        const int cs = j & 1;
        if (j + 1 < CK) {
            rd16(kk[cs ^ 1], kr + (j + 1) * FROW);
            rd16(qq[cs ^ 1], qr + (j + 1) * FROW);
            gg[cs ^ 1] = *reinterpret_cast<const float4*>(gt + (j + 1) * 8);
        }
        if (SC && (j & 3) == 0) gs = *reinterpret_cast<const float2*>(gt + (p + j) * 8 + 4);
        if (j < FR / 4)
            *reinterpret_cast<float4*>(ckdst + 4 * j) = make_float4(ck[4 * j], ck[4 * j + 1], ck[4 * j + 2], ck[4 * j + 3]);
        // one wave per SIMD: nothing else hides LDS latency, so the reads of
        // step j + 1 stay at the top of step j, a whole step ahead of their use
        __builtin_amdgcn_sched_barrier(0);
        const float4 g = gg[cs];
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int m = 0; m < FR; m += 2) {
            a0 = fmaf(s[m], kk[cs][m], a0);
            a1 = fmaf(s[m + 1], kk[cs][m + 1], a1);
        }
        const float x = group_sum<4>(a0 + a1);
        float o0 = 0.0f, o1 = 0.0f;
        if constexpr (SC) {
            const float ut = g.x * fmaf(vv[j], g.y, -x);
#pragma unroll
            for (int m = 0; m < FR; m += 2) {
                s[m] = fmaf(kk[cs][m], ut, s[m]);
                s[m + 1] = fmaf(kk[cs][m + 1], ut, s[m + 1]);
                o0 = fmaf(s[m], qq[cs][m], o0);
                o1 = fmaf(s[m + 1], qq[cs][m + 1], o1);
            }
        } else {
            const float a = g.z;
            const float u = g.x * (vv[j] - a * x);
#pragma unroll
            for (int m = 0; m < FR; m += 2) {
                s[m] = a * s[m] + kk[cs][m] * u;
                s[m + 1] = a * s[m + 1] + kk[cs][m + 1] * u;
                o0 = fmaf(s[m], qq[cs][m], o0);
                o1 = fmaf(s[m + 1], qq[cs][m + 1], o1);
            }
        }
        const float oo = group_sum<4>(o0 + o1);
        const bool mine = p == (j & 3);
        ho = mine ? oo : ho;
        hs = mine ? x : hs;
        if ((j & 3) == 3 && j + 1 < CK) {
            const int jj = p + (j & ~3);
            const bool ok = jj < nvalid;
            *(ok ? od + jj * d : tr) = SC ? ho * gs.x : ho;
            *(ok ? skd + jj * d : tr + 1) = SC ? hs * gs.y : hs;
        }
        if (j + 1 == CK) {
            last_o = SC ? ho * gs.x : ho;
            last_sk = SC ? hs * gs.y : hs;
        }
    }
}

ASCA_DEV void store_state(float* __restrict__ dst, const float (&s)[FR]) {
#pragma unroll
    for (int e = 0; e < FR; e += 4)
        *reinterpret_cast<float4*>(dst + e) = make_float4(s[e], s[e + 1], s[e + 2], s[e + 3]);
}

// One block per unit = h*B + b (the reference's s_pre order,
// rust/src/delta.rs:54-56).
template <bool AL>
__global__ __launch_bounds__(NT) void delta_fwd64_k(const float* __restrict__ q, const float* __restrict__ k,
                                                    const float* __restrict__ v, const float* __restrict__ alpha,
                                                    const float* __restrict__ beta, float* __restrict__ o,
                                                    float* __restrict__ sk_out, float* __restrict__ ckpt, int B,
                                                    int T, int H, int nslots) {
    __shared__ float4 lds4[2 * F_BUF / 4];
    float* const lds = reinterpret_cast<float*>(lds4);
    const int unit = blockIdx.x;
    const int h = unit / B, b = unit - h * B;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int c = lane >> 2, p = lane & 3;
    const int col = 16 * w + c;
    const long d = (long)H * DH;
    const long ubase = (long)b * T * d + (long)h * DH;
    const long gbase = (long)b * T * H + h;
    float* const ckb = ckpt + (long)unit * nslots * DH2 + col * DH + 16 * p;
    float* const tr = trash(threadIdx.x * 8);
    const int nchunk = (T + CK - 1) / CK;

    float s[FR];
#pragma unroll
    for (int m = 0; m < FR; ++m) s[m] = 0.0f;

    // Staged loads run two chunks ahead (the loads of chunk ci + 2 are queued
    // at the start of chunk ci, into the register set that chunk ci + 1's data
    // has just left for LDS), so each has two chunks of compute to arrive.
    FStage sa, sb;
    fstage_load<AL>(sa, 0, q, k, v, alpha, beta, ubase, gbase, d, T, H, lane);
    bool sc_next = fstage_store(sa, lds, w, lane);
    fstage_load<AL>(sa, min(1, nchunk - 1), q, k, v, alpha, beta, ubase, gbase, d, T, H, lane);
    lds_barrier();

    // the last output group of the previous chunk, stored after this chunk's loads
    float* pend_o = tr;
    float* pend_sk = tr + 1;
    float last_o = 0.0f, last_sk = 0.0f;
    // chunk ci: `cur` holds chunk ci + 1 (stored to LDS at the end), `nxt` is
    // loaded with chunk ci + 2
    auto chunk = [&](int ci, FStage& cur, FStage& nxt) {
        const int t0 = ci * CK;
        const float* const buf = lds + (ci & 1) * F_BUF;
        const float* const gt = buf + F_G + w * CK * 8;
        const bool sc = sc_next;
        fstage_load<AL>(nxt, min(ci + 2, nchunk - 1), q, k, v, alpha, beta, ubase, gbase, d, T, H, lane);
        *pend_o = last_o;
        *pend_sk = last_sk;
        float vv[CK];
#pragma unroll
        for (int j = 0; j < CK; ++j) vv[j] = buf[F_V + j * DH + col];
        float ck[FR];   // the checkpoint: S before step t0
#pragma unroll
        for (int m = 0; m < FR; ++m) ck[m] = s[m];
        float* const od = o + ubase + (long)t0 * d + col;
        float* const skd = sk_out + ubase + (long)t0 * d + col;
        if (sc) {
            fsteps<true>(s, buf, gt, vv, p, ck, ckb + (long)ci * DH2, od, skd, d, T - t0, tr, last_o, last_sk);
            const float ge = gt[(CK - 1) * 8 + 4];
#pragma unroll
            for (int m = 0; m < FR; ++m) s[m] *= ge;
        } else {
            fsteps<false>(s, buf, gt, vv, p, ck, ckb + (long)ci * DH2, od, skd, d, T - t0, tr, last_o, last_sk);
        }
        {
            const int jj = p + CK - 4;
            const bool ok = jj < T - t0;
            pend_o = ok ? od + jj * d : tr;
            pend_sk = ok ? skd + jj * d : tr + 1;
        }
        sc_next = fstage_store(cur, lds + ((ci + 1) & 1) * F_BUF, w, lane);
        lds_barrier();
    };
    for (int ci = 0; ci < nchunk; ci += 2) {
        chunk(ci, sa, sb);
        if (ci + 1 < nchunk) chunk(ci + 1, sb, sa);
    }
    *pend_o = last_o;
    *pend_sk = last_sk;
    store_state(ckb + (long)nchunk * DH2, s);   // the state after step T-1
}

// ================================================================= backward

constexpr int BM = 8;                       // rows per lane (two columns each)
constexpr int BROW = 72;                    // padded q / k row: rows 32..63 shifted by 4 floats
ASCA_DEV int bpad(int a) { return a + 4 * (a >> 5); }
constexpr int RROW = 68;                    // reduction row buffer, same padding
// Segment buffer (floats): per-step dq / dk row sums of each wave, the dalpha /
// dbeta totals, the dv rows, the staged q and k rows, each wave's dO, v, sk
// columns, the gate table (row j = alpha, beta, G_{j+1}, 1/G_{j+1}, 1/alpha,
// |q|, |k|, beta/G_{j+1}) with the segment's range flag, and a sink.
constexpr int B_RQ = 0;                          // [CK][W][RROW]
constexpr int B_RK = B_RQ + CK * W * RROW;       // [CK][W][RROW]
constexpr int B_RAB = B_RK + CK * W * RROW;      // [CK][W][2]
constexpr int B_RV = B_RAB + CK * W * 2;         // [CK][DH]
constexpr int B_Q = B_RV + CK * DH;              // [CK][BROW]
constexpr int B_K = B_Q + CK * BROW;             // [CK][BROW]
constexpr int B_W = B_K + CK * BROW;             // [W][CK][3][16]
constexpr int B_G = B_W + W * CK * 48;           // [CK][8], flag at + 8 CK
constexpr int B_SINK = B_G + 8 * CK + 4;
constexpr int B_BUF = B_SINK + 8;
static_assert(B_BUF % 4 == 0 && B_Q % 4 == 0 && B_W % 4 == 0 && B_G % 4 == 0, "float4 buffers");
// After the two segment buffers: the next segment's end-state tile, 16 floats
// per thread as [4][NT] float4.
constexpr size_t B_LDS = (2 * (size_t)B_BUF + 16 * NT) * 4;
static_assert(B_LDS <= 160 * 1024, "backward LDS");

// (vectors first: a scalar member ahead of the float4 array kept the compiler
// from promoting the whole struct to registers)
struct BStage {
    float4 rq[2];    // two float4 of the segment's q or k rows
    float4 rw[3];    // the wave's dO, v, sk columns (192 float4 over 64 lanes)
    float4 rck[4];   // end-state tile: column colb + n, rows rowb + 4 hf .. (index 2n + hf)
    float rab;       // lane j < CK: alpha of step j; CK <= j < 2CK: beta (as loaded)
    float rqk;       // the same lanes: |q|, |k| (fused backward)
};

template <bool FUSED, bool AL>
ASCA_DEV void bstage_load(BStage& st, int g, const float* __restrict__ q, const float* __restrict__ k,
                          const float* __restrict__ v, const float* __restrict__ d_o,
                          const float* __restrict__ skv, const float* __restrict__ alpha,
                          const float* __restrict__ beta, const float* __restrict__ qnorm,
                          const float* __restrict__ knorm, const float* __restrict__ ckb, long ubase, long gbase,
                          long d, int T, int H, int w, int lane, int rowb, int colb) {
    const int t0 = g * CK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int f = threadIdx.x + NT * i;
        const int tsr = f >> 8, j = (f >> 4) & (CK - 1), c4 = f & 15;
        const long t = min(t0 + j, T - 1);
        st.rq[i] = ld4<AL>((tsr ? k : q) + ubase + t * d + 4 * c4);
    }
    // tensor i: 0 dO, 1 v, 2 sk (the workspace's, always aligned)
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int j = lane >> 2, q4 = lane & 3;
        const long t = min(t0 + j, T - 1);
        const long o = ubase + t * d + 16 * w + 4 * q4;
        st.rw[i] = i == 0 ? ld4<AL>(d_o + o) : (i == 1 ? ld4<AL>(v + o) : ld4<true>(skv + o));
    }
    {
        const int gl = lane & (2 * CK - 1);
        const int t = t0 + (gl & (CK - 1));
        const long tc = min(t, T - 1);
        // raw values: bstage_store applies the padding past T, so these loads
        // never turn into loads under a lane condition
        (void)t;
        st.rab = (gl < CK ? alpha : beta)[gbase + tc * H];
        st.rqk = FUSED ? (gl < CK ? qnorm : knorm)[gbase + tc * H] : 0.0f;
    }
    const float* const ce = ckb + (long)(g + 1) * DH2;   // the state after the segment
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
            st.rck[2 * n + hf] = *reinterpret_cast<const float4*>(ce + (long)(colb + n) * DH + rowb + 4 * hf);
}

// Registers -> the buffer nb of segment g and this thread's end-state slot.
// Every lane stores, lanes without an element into the sink, so no staged load
// is ever moved down next to a conditional store.  Padded steps get dO = 0.
ASCA_DEV void bstage_store(const BStage& st, int g, int T, float* __restrict__ nb, float4* __restrict__ cks,
                           int w, int lane) {
    float* const sink = nb + B_SINK;
#pragma unroll
    for (int i = 0; i < 4; ++i) cks[i * NT] = st.rck[i];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int f = threadIdx.x + NT * i;
        const int tsr = f >> 8, j = (f >> 4) & (CK - 1), c4 = f & 15;
        *reinterpret_cast<float4*>(nb + (tsr ? B_K : B_Q) + j * BROW + bpad(4 * c4)) = st.rq[i];
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int j = lane >> 2, q4 = lane & 3;
        float4 x = st.rw[i];
        if (i == 0 && g * CK + j >= T) x = make_float4(0.f, 0.f, 0.f, 0.f);
        *reinterpret_cast<float4*>(nb + B_W + ((w * CK + j) * 3 + i) * 16 + 4 * q4) = x;
    }
    // Gate table, written by wave 0 (the other waves compute into the sink).
    // Lanes j < CK hold alpha_j, lanes CK + j hold beta_j.
    // Lane j < CK writes alpha_j, G_{j+1}, 1/G_{j+1}, 1/alpha_j, |q_j| into row j;
    // lane CK + j writes beta_j, beta_j / G_{j+1}, |k_j| into row j.
    // The callers (the scaled and the plain segment) both store here; without
    // this opaque copy the compiler hoists the identical gate arithmetic of the
    // two into the segment's start, right behind the loads it waits for.
    float rab = st.rab, rqk = st.rqk;
    asm volatile("" : "+v"(rab), "+v"(rqk));
    const bool w0 = w == 0;
    const bool ga = lane < CK;
    const bool gb = lane >= CK && lane < 2 * CK;
    // steps past T: alpha = 1, beta = 0 leave the state unchanged
    if (g * CK + (lane & (CK - 1)) >= T) rab = ga ? 1.0f : 0.0f;
    const float pr = prefix_prod<CK>(ga ? rab : 1.0f);   // lane j < CK: G_{j+1}
    const float prb = __shfl(pr, lane & (CK - 1));           // lane CK + j: G_{j+1}
    float* const row = (w0 && (ga || gb)) ? nb + B_G + (lane & (CK - 1)) * 8 : sink;
    float* const rowa = (w0 && ga) ? row : sink;
    row[ga ? 0 : 1] = rab;
    row[ga ? 2 : 7] = ga ? pr : rab * __builtin_amdgcn_rcpf(prb);
    row[ga ? 3 : 6] = ga ? __builtin_amdgcn_rcpf(pr) : rqk;
    rowa[4] = __builtin_amdgcn_rcpf(rab);
    rowa[5] = rqk;
    // The scaled walk runs backwards: stepping s_j back to s_{j-1} magnifies
    // rounding by 1/alpha_j, so over the segment by up to 1/prod(min(alpha, 1)).
    // It is taken when that product is at least 2^-8 and every alpha lies in
    // [2^-7, 2^7] (G within 2^+-112); other segments recompute their states
    // forwards.
    const float pm = prefix_prod<CK>(ga ? fminf(rab, 1.0f) : 1.0f);
    const float amp = readlane_f(pm, CK - 1);
    const bool bad = ga && !(rab >= 0x1p-7f && rab <= 0x1p7f);
    const bool in_range = __ballot(bad) == 0 && amp >= 0x1p-8f;
    *(w0 && lane == 0 ? nb + B_G + 8 * CK : sink + 3) = in_range ? 1.0f : 0.0f;
}

struct BOps {
    float q[BM], k[BM];
    float2 dO, v, sk;
    float a, b, g1, r1, ia, cu;   // alpha, beta, G_{j+1}, 1/G_{j+1}, 1/alpha, beta/G_{j+1}
};

ASCA_DEV void bops_read(BOps& o, const float* __restrict__ buf, int j, int w, int rowb, int cg) {
    const float* const qr = buf + B_Q + j * BROW + bpad(rowb);
    const float* const kr = buf + B_K + j * BROW + bpad(rowb);
#pragma unroll
    for (int e = 0; e < BM; e += 4) {
        const float4 x = *reinterpret_cast<const float4*>(qr + e);
        const float4 y = *reinterpret_cast<const float4*>(kr + e);
        o.q[e] = x.x; o.q[e + 1] = x.y; o.q[e + 2] = x.z; o.q[e + 3] = x.w;
        o.k[e] = y.x; o.k[e + 1] = y.y; o.k[e + 2] = y.z; o.k[e + 3] = y.w;
    }
    const float* const sw = buf + B_W + (w * CK + j) * 48 + 2 * cg;
    o.dO = *reinterpret_cast<const float2*>(sw);
    o.v = *reinterpret_cast<const float2*>(sw + 16);
    o.sk = *reinterpret_cast<const float2*>(sw + 32);
    const float4 g0 = *reinterpret_cast<const float4*>(buf + B_G + 8 * j);
    const float4 g1 = *reinterpret_cast<const float4*>(buf + B_G + 8 * j + 4);
    o.a = g0.x;
    o.b = g0.y;
    o.g1 = g0.z;
    o.r1 = g0.w;
    o.ia = g1.x;
    o.cu = g1.w;
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

ASCA_DEV int rpad(int r) { return r + 4 * (r >> 5); }

// One reverse step for this lane's 8 x 2 tile (rust/src/delta.rs:485-572 per
// element).  sa: the state after the step; sm: the state before it.
//   SC = true: sa = S_j / G_{j+1}, sm = S_{j-1} / G_j, ds = G_{j+1} dS; the step
//     derives sm from sa in place (s) and every output term takes its scale from
//     the gate row.
//   SC = false: s holds S_j on entry, sm is given, ds = dS.
//   first: the step is the first of its sequence, whose previous state is
//     exactly zero (the scaled walk would leave rounding residue there).
template <bool SC>
ASCA_DEV void bstep(const BOps& in, float (&s)[BM][2], const float (&smp)[BM][2], float (&ds)[BM][2],
                    float* __restrict__ rq, float* __restrict__ rk, float* __restrict__ rv, float& pab_out,
                    int lane, int rg, int colb, bool first = false) {
    float dO0 = in.dO.x, dO1 = in.dO.y;
    if constexpr (SC) {
        dO0 *= in.g1;
        dO1 *= in.g1;
    }
    // dS += q dO^T  (delta.rs:508-511)
#pragma unroll
    for (int m = 0; m < BM; ++m) {
        ds[m][0] = fmaf(in.q[m], dO0, ds[m][0]);
        ds[m][1] = fmaf(in.q[m], dO1, ds[m][1]);
    }
    // du = dS^T k  (delta.rs:536-542): 8-lane butterfly over the row groups
    float c0 = 0.0f, c1 = 0.0f;
#pragma unroll
    for (int m = 0; m < BM; ++m) {
        c0 = fmaf(ds[m][0], in.k[m], c0);
        c1 = fmaf(ds[m][1], in.k[m], c1);
    }
    const float dt0 = group_sum<8>(c0), dt1 = group_sum<8>(c1);
    const float du0 = SC ? dt0 * in.r1 : dt0, du1 = SC ? dt1 * in.r1 : dt1;
    const float wv0 = fmaf(-in.a, in.sk.x, in.v.x), wv1 = fmaf(-in.a, in.sk.y, in.v.y);
    // uh: the u that multiplies dS (u~ = u / G_{j+1} when scaled); sh: the dsk
    // that multiplies S_{j-1} and updates dS (G_j dsk when scaled)
    const float cu = SC ? in.cu : in.b;
    const float uh0 = cu * wv0, uh1 = cu * wv1;
    const float cs = SC ? -in.b : -in.b * in.a;
    const float sh0 = cs * dt0, sh1 = cs * dt1;
    // dv = beta du  (delta.rs:550), one LDS row per step
    if (rg == 0) *reinterpret_cast<float2*>(rv + colb) = make_float2(in.b * du0, in.b * du1);

    // dq = S_j dO  (delta.rs:504-507)
    float pq[BM], pk[BM];
#pragma unroll
    for (int m = 0; m < BM; ++m) pq[m] = fmaf(s[m][1], dO1, s[m][0] * dO0);
    if constexpr (SC) {
        // back one step: s = S_{j-1} / G_j
#pragma unroll
        for (int m = 0; m < BM; ++m) {
            s[m][0] = fmaf(-in.k[m], uh0, s[m][0]);
            s[m][1] = fmaf(-in.k[m], uh1, s[m][1]);
        }
        if (first) {
#pragma unroll
            for (int m = 0; m < BM; ++m) s[m][0] = s[m][1] = 0.0f;
        }
    }
    // sm: S_{j-1} (scaled: the caller passes s itself, now stepped back)
    const float (&sm)[BM][2] = smp;
    //   dk = dS u + S_{j-1} dsk    (delta.rs:532-534, 556-558)
    //   dalpha = <dS, S_{j-1}> - beta du.sk ; dbeta = du.(v - alpha sk)   (:530, 548-553)
    float pa0 = 0.0f, pa1 = 0.0f;
#pragma unroll
    for (int m = 0; m < BM; ++m) {
        float x = uh0 * ds[m][0];
        x = fmaf(uh1, ds[m][1], x);
        x = fmaf(sh0, sm[m][0], x);
        pk[m] = fmaf(sh1, sm[m][1], x);
        pa0 = fmaf(ds[m][0], sm[m][0], pa0);
        pa1 = fmaf(ds[m][1], sm[m][1], pa1);
    }
    const float ea = -in.b * fmaf(du1, in.sk.y, du0 * in.sk.x);
    const float eb = fmaf(du1, wv1, du0 * wv0);
    const float pab = SC ? (pa0 + pa1) * in.ia : pa0 + pa1;
    const float pa = pab + (rg == 0 ? ea : 0.0f);
    const float pb = rg == 0 ? eb : 0.0f;
    // dS <- alpha dS + k dsk^T  (delta.rs:543-545, 559-563)
#pragma unroll
    for (int m = 0; m < BM; ++m) {
        if constexpr (SC) {
            ds[m][0] = fmaf(in.k[m], sh0, ds[m][0]);
            ds[m][1] = fmaf(in.k[m], sh1, ds[m][1]);
        } else {
            ds[m][0] = in.a * ds[m][0] + in.k[m] * sh0;
            ds[m][1] = in.a * ds[m][1] + in.k[m] * sh1;
        }
    }
    const int r = rpad(8 * (lane & 7) + (lane >> 3));
    rq[r] = colsum8(pq, lane);
    rk[r] = colsum8(pk, lane);
    pab_out = tsum32(pa, pb);
}

// S_{j} from S_{j-1} (rust/src/delta.rs:299-306), for the recompute of a plain
// segment.
ASCA_DEV void fwd_update(float (&x)[BM][2], const float* __restrict__ buf, int j, int w, int rowb, int cg) {
    const float* const kr = buf + B_K + j * BROW + bpad(rowb);
    const float* const sw = buf + B_W + (w * CK + j) * 48 + 2 * cg;
    const float2 vv = *reinterpret_cast<const float2*>(sw + 16);
    const float2 sk = *reinterpret_cast<const float2*>(sw + 32);
    const float a = buf[B_G + 8 * j], bt = buf[B_G + 8 * j + 1];
    const float u0 = bt * (vv.x - a * sk.x), u1 = bt * (vv.y - a * sk.y);
#pragma unroll
    for (int e = 0; e < BM; e += 4) {
        const float4 kk = *reinterpret_cast<const float4*>(kr + e);
        const float km[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[e + i][0] = a * x[e + i][0] + km[i] * u0;
            x[e + i][1] = a * x[e + i][1] + km[i] * u1;
        }
    }
}

// One scaled segment in reverse (every gate of the segment in [2^-8, 2^8]).
// se: this thread's tile of the state after the segment; ds enters and leaves
// unscaled.  The next segment's staged operands are stored into nb halfway.
ASCA_DEV void bsegment_sc(const float (&se)[BM][2], float (&ds)[BM][2], const BStage& stg, int g, int T,
                          float* __restrict__ buf, float* __restrict__ nb, float4* __restrict__ cks, int w,
                          int lane, int rg, int cg, int rowb, int colb) {
    float s[BM][2];
    const float rend = buf[B_G + 8 * (CK - 1) + 3];   // 1 / G_CK
    const float gend = buf[B_G + 8 * (CK - 1) + 2];   // G_CK
#pragma unroll
    for (int m = 0; m < BM; ++m) {
        s[m][0] = se[m][0] * rend;
        s[m][1] = se[m][1] * rend;
        ds[m][0] *= gend;
        ds[m][1] *= gend;
    }
    float pab[CK];
    BOps op[2];
    bops_read(op[(CK - 1) & 1], buf, CK - 1, w, rowb, cg);
#pragma unroll
    for (int jj = CK - 1; jj >= 0; --jj) {
        if (jj > 0) bops_read(op[(jj - 1) & 1], buf, jj - 1, w, rowb, cg);
        // the operand reads of the next step stay a whole step ahead of their use
        __builtin_amdgcn_sched_barrier(0);
        bstep<true>(op[jj & 1], s, s, ds, buf + B_RQ + jj * W * RROW + w * RROW,
                    buf + B_RK + jj * W * RROW + w * RROW, buf + B_RV + jj * DH, pab[jj], lane, rg, colb,
                    jj == 0 && g == 0);
        if (jj == CK / 2) {
            // the staged operands of the next segment (loads issued at this
            // segment's start) go to its buffer; the fence keeps the scheduler
            // from hoisting the stores, and their wait, to the segment's start
            __builtin_amdgcn_sched_barrier(0);
            bstage_store(stg, g > 0 ? g - 1 : 0, T, nb, cks, w, lane);
        }
    }
    cross_step_sum<CK, W>(pab, buf + B_RAB, w, lane);
}

// One plain segment in reverse (some gate of the segment outside [2^-8, 2^8]:
// zeros, tiny or huge values).  Each step recomputes S_{j-1} and S_j from the
// segment's first checkpoint, so no division by a gate occurs; a rolled loop,
// since these segments are rare and their registers must not raise the
// kernel's budget.
ASCA_DEV void bsegment_plain(float (&ds)[BM][2], const BStage& stg, int g, int T, float* __restrict__ buf,
                             float* __restrict__ nb, float4* __restrict__ cks, const float* __restrict__ ckb,
                             int w, int lane, int rg, int cg, int rowb, int colb) {
    float st0[BM][2];
    const float* const cs = ckb + (long)g * DH2;
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const float4 x = *reinterpret_cast<const float4*>(cs + (long)(colb + n) * DH + rowb + 4 * hf);
            st0[4 * hf][n] = x.x;
            st0[4 * hf + 1][n] = x.y;
            st0[4 * hf + 2][n] = x.z;
            st0[4 * hf + 3][n] = x.w;
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
        for (int i = 0; i < jj; ++i) fwd_update(sm, buf, i, w, rowb, cg);
#pragma unroll
        for (int m = 0; m < BM; ++m) {
            s[m][0] = sm[m][0];
            s[m][1] = sm[m][1];
        }
        fwd_update(s, buf, jj, w, rowb, cg);
        BOps op;
        bops_read(op, buf, jj, w, rowb, cg);
        float pab;
        bstep<false>(op, s, sm, ds, buf + B_RQ + jj * W * RROW + w * RROW, buf + B_RK + jj * W * RROW + w * RROW,
                     buf + B_RV + jj * DH, pab, lane, rg, colb);
        // lanes < 32 hold dalpha pair sums, lanes >= 32 dbeta ones
        const float tot = add_xor16(group_sum<16>(pab));
        if ((lane & 31) == 0) buf[B_RAB + (jj * W + w) * 2 + (lane >> 5)] = tot;
    }
    // after the loop, not inside it under a condition: every path then provably
    // waits for the staged loads here, and no later reuse of their registers does
    bstage_store(stg, g > 0 ? g - 1 : 0, T, nb, cks, w, lane);
}

template <bool FUSED, bool AL>
__global__ __launch_bounds__(NT) void delta_bwd64_k(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ alpha, const float* __restrict__ beta, const float* __restrict__ d_o,
    const float* __restrict__ skv, const float* __restrict__ ckpt, const float* __restrict__ qnorm,
    const float* __restrict__ knorm, float* __restrict__ gq, float* __restrict__ gk, float* __restrict__ gv,
    long ldx, float* __restrict__ ga, float* __restrict__ gb, long ldg, int B, int T, int H, int nslots) {
    extern __shared__ float4 lds4[];
    float* const lds = reinterpret_cast<float*>(lds4);
    float4* const cks = lds4 + 2 * B_BUF / 4 + threadIdx.x;

    const int unit = blockIdx.x;
    const int h = unit / B, b = unit - h * B;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int rg = lane & 7, cg = lane >> 3;
    const int colb = 16 * w + 2 * cg;
    const int rowb = BM * rg;
    const long d = (long)H * DH;
    const long ubase = (long)b * T * d + (long)h * DH;
    const long gbase = (long)b * T * H + h;
    const long hoff = (long)h * DH;
    const float* const ckb = ckpt + (long)unit * nslots * DH2;
    const int nseg = (T + CK - 1) / CK;

    float ds[BM][2];
#pragma unroll
    for (int m = 0; m < BM; ++m) ds[m][0] = ds[m][1] = 0.0f;

    BStage stg;
    bstage_load<FUSED, AL>(stg, nseg - 1, q, k, v, d_o, skv, alpha, beta, qnorm, knorm, ckb, ubase, gbase, d, T, H, w,
                       lane, rowb, colb);
    bstage_store(stg, nseg - 1, T, lds + ((nseg - 1) & 1) * B_BUF, cks, w, lane);

    for (int g = nseg - 1; g >= 0; --g) {
        const int t0 = g * CK;
        float* const buf = lds + (g & 1) * B_BUF;
        float* const nb = lds + ((g + 1) & 1) * B_BUF;   // the next segment's (g - 1)
        float se[BM][2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 x = cks[i * NT];   // index 2n + hf: column n, rows 4hf..4hf+3
            const int n = i >> 1, hf = i & 1;
            se[4 * hf][n] = x.x;
            se[4 * hf + 1][n] = x.y;
            se[4 * hf + 2][n] = x.z;
            se[4 * hf + 3][n] = x.w;
        }
        bstage_load<FUSED, AL>(stg, g > 0 ? g - 1 : 0, q, k, v, d_o, skv, alpha, beta, qnorm, knorm, ckb, ubase, gbase,
                           d, T, H, w, lane, rowb, colb);
        lds_barrier();   // this segment's staging visible to all waves

        if (__builtin_amdgcn_readfirstlane(__float_as_int(buf[B_G + 8 * CK])) == __float_as_int(1.0f))
            bsegment_sc(se, ds, stg, g, T, buf, nb, cks, w, lane, rg, cg, rowb, colb);
        else
            bsegment_plain(ds, stg, g, T, buf, nb, cks, ckb, w, lane, rg, cg, rowb, colb);
        lds_barrier();   // this segment's row sums complete

        // cross-wave sums, fused norm / sigmoid backward, stores: wave w takes
        // steps w + W i, lane = row.  Every LDS read of the wave's steps is
        // issued before the arithmetic and the stores (steps past T only skip
        // their stores), so the reads' latency is paid once per segment.
        constexpr int NS = CK / W;
        const int a = lane;
        float dq[NS], dk[NS], dA[NS], dB[NS], dvv[NS], qa[NS], ka[NS], nq[NS], nk[NS], al[NS], be[NS];
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const int jj = w + W * i;
            const float* const rq = buf + B_RQ + jj * W * RROW + rpad(a);
            const float* const rk = buf + B_RK + jj * W * RROW + rpad(a);
            const float* const rab = buf + B_RAB + jj * W * 2;
            dq[i] = (rq[0] + rq[RROW]) + (rq[2 * RROW] + rq[3 * RROW]);
            dk[i] = (rk[0] + rk[RROW]) + (rk[2 * RROW] + rk[3 * RROW]);
            dA[i] = (rab[0] + rab[2]) + (rab[4] + rab[6]);
            dB[i] = (rab[1] + rab[3]) + (rab[5] + rab[7]);
            dvv[i] = buf[B_RV + jj * DH + a];
            qa[i] = buf[B_Q + jj * BROW + bpad(a)];
            ka[i] = buf[B_K + jj * BROW + bpad(a)];
            nq[i] = buf[B_G + 8 * jj + 5];
            nk[i] = buf[B_G + 8 * jj + 6];
            al[i] = buf[B_G + 8 * jj];
            be[i] = buf[B_G + 8 * jj + 1];
        }
        static_assert(W == 4, "the cross-wave sums above add four waves");
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const int jj = w + W * i;
            if (t0 + jj >= T) continue;   // wave-uniform
            const long r = (long)b * T + t0 + jj;
            gv[r * ldx + hoff + a] = dvv[i];
            if constexpr (FUSED) {
                const float dotq = wave_sum(qa[i] * dq[i]);
                const float dotk = wave_sum(ka[i] * dk[i]);
                // 1/|q|, 1/|k| by the hardware reciprocal (within 1 ulp)
                gq[r * ldx + hoff + a] = (dq[i] - qa[i] * dotq) * __builtin_amdgcn_rcpf(nq[i]);
                gk[r * ldx + hoff + a] = (dk[i] - ka[i] * dotk) * __builtin_amdgcn_rcpf(nk[i]);
                if (lane == 0) {
                    ga[r * ldg + h] = dA[i] * al[i] * (1.0f - al[i]);
                    gb[r * ldg + h] = dB[i] * be[i] * (1.0f - be[i]);
                }
            } else {
                gq[r * ldx + hoff + a] = dq[i];
                gk[r * ldx + hoff + a] = dk[i];
                if (lane == 0) {
                    ga[r * ldg + h] = dA[i];
                    gb[r * ldg + h] = dB[i];
                }
            }
        }
    }
}

}  // namespace d64

template <bool AL>
static int launch_fwd64_t(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                          float* o, const DeltaWs& ws, int B, int T, int H, hipStream_t st) {
    int rc = pre_launch("delta_fwd64");
    if (rc) return rc;
    hipLaunchKernelGGL(d64::delta_fwd64_k<AL>, dim3(B * H), dim3(d64::NT), 0, st, q, k, v, alpha, beta, o, ws.sk,
                       ws.ckpt, B, T, H, ws.nslots);
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
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)d64::B_LDS);
        if (e != hipSuccess)
            return fail(ASCA_ERR_HIP, "hipFuncSetAttribute(LDS %zu): %s", d64::B_LDS, hipGetErrorString(e));
        attr = true;
    }
    int rc = pre_launch("delta_bwd64");
    if (rc) return rc;
    hipLaunchKernelGGL((d64::delta_bwd64_k<FUSED, AL>), dim3(B * H), dim3(d64::NT), d64::B_LDS, st, q, k, v, alpha,
                       beta, d_o, ws.sk, ws.ckpt, qn, kn, gq, gk, gv, ldx, ga, gb, ldg, B, T, H, ws.nslots);
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
