// Gated delta rule at dh = 64, f32, blocked (UT) form: the forward and the
// fused backward on 16-byte-aligned rows (the configs[1] / training hot path).
// The kernels are in ut64_kernels.h; the other backward variants are launched
// from delta_ut64_b.hip.
#include "ut64_kernels.h"

namespace asca {

int launch_ut_fwd64(const float* q, const float* k, const float* v, const float* alpha, const float* beta, float* o,
                    const DeltaWs& ws, int B, int T, int H, hipStream_t st) {
    if (ws.ck != D64_CK || ws.cs != 1) return fail(ASCA_ERR_INVALID, "ut_fwd64: workspace layout mismatch");
    // the buffer resources over a unit's rows, gates, u tiles, checkpoints and
    // records take 32-bit byte sizes and offsets
    const long NC = (T + ut64::C - 1) / ut64::C;
    if ((long)T * H * ut64::DH >= (1L << 30) || (long)T * H >= (1L << 30) || (NC + 1) * ut64::DH2 >= (1L << 30) ||
        NC * ut64::R_SZ >= (1L << 30))
        return fail(ASCA_ERR_UNSUPPORTED, "ut_fwd64: one sequence's rows exceed 32-bit byte offsets");
    return ut_aligned16(q) && ut_aligned16(k) && ut_aligned16(v) && ut_aligned16(o)
               ? launch_ut_fwd64_t<true>(q, k, v, alpha, beta, o, ws, B, T, H, st)
               : launch_ut_fwd64_t<false>(q, k, v, alpha, beta, o, ws, B, T, H, st);
}

int launch_ut_bwd64(bool fused, const float* q, const float* k, const float* v, const float* alpha,
                    const float* beta, const float* d_o, const DeltaWs& ws, const float* qn, const float* kn,
                    float* gq, float* gk, float* gv, long ldx, float* ga, float* gb, long ldg, int B, int T, int H,
                    hipStream_t st) {
    if (ws.cs != 1 || !ws.rec) return fail(ASCA_ERR_INVALID, "ut_bwd64: workspace layout mismatch");
    ut64::BArgs a;
    a.q = q; a.k = k; a.v = v; a.alpha = alpha; a.beta = beta; a.d_o = d_o; a.u = ws.sk; a.ckpt = ws.ckpt;
    a.rec = ws.rec; a.qn = qn; a.kn = kn; a.gq = gq; a.gk = gk; a.gv = gv; a.ga = ga; a.gb = gb;
    a.ldx = ldx; a.ldg = ldg; a.d = (long)H * ut64::DH; a.T = T; a.H = H; a.nslots = ws.nslots;
    a.NC = (T + ut64::C - 1) / ut64::C;
    // per-unit fields are filled in the kernel from blockIdx
    const bool al = ut_aligned16(q) && ut_aligned16(k) && ut_aligned16(v) && ut_aligned16(d_o) && ut_aligned16(gq) &&
                    ut_aligned16(gk) && ut_aligned16(gv) && (ldx * 4) % 16 == 0;
    const int units = B * H;
    a.B = B; a.unit = 0; a.h = 0; a.ubase = 0; a.gbase = 0; a.rowbase = 0;
    // element offsets within a unit are 32-bit, and the buffer resources over a
    // unit's rows, checkpoints and records take 32-bit byte sizes and offsets
    if ((long)T * (ldx > a.d ? ldx : a.d) >= (1L << 30) || (long)T * ldg >= (1L << 30) ||
        (long)((T + ut64::C - 1) / ut64::C + 1) * ut64::DH2 >= (1L << 30) ||
        (long)((T + ut64::C - 1) / ut64::C) * ut64::R_SZ >= (1L << 30))
        return fail(ASCA_ERR_UNSUPPORTED, "ut_bwd64: one sequence's rows exceed 32-bit byte offsets");
    a.di = (int)a.d; a.ldxi = (int)ldx; a.ldgi = (int)ldg;
    // the gate sums: scratch of this call on its stream (the forward's workspace is only read)
    StreamScratch sc;
    int rc = sc.get(ut_bwd64_scratch_floats(units, a.NC), st);
    if (rc) return rc;
    a.gsc = sc.ws.p;
    rc = fused && al ? launch_ut_bwd64_t<true, true>(a, units, st) : launch_ut_bwd64_other(a, units, fused, al, st);
    const int rr = sc.release(st);
    return rc ? rc : rr;
}

}  // namespace asca
