// Hash-routed mixture of experts, forward and backward, all on the device.
//
// Tokens are bucketed by expert with asca_hash_route (perm = tokens sorted by
// expert, stable; offsets = CSR bounds).  Every per-expert product of the
// reference (Gpu::moe_forward_dev, rust/src/cuda/mod.rs:523-607, and
// Gpu::moe_bwd_dev, mod.rs:745-824, over the CPU semantics of HashMoe::forward
// / backward, rust/src/model.rs:187-306 and :339-497) becomes ONE grouped MFMA
// GEMM launch over all experts, with the row gather fused into the operand
// loads, the row scatter into the stores, and bias / SiLU / SiLU-backward in
// the epilogues.  No host synchronisation: group sizes stay on the device.
//
// Layouts (row-major f32): xn, out, dout, dxn (T x d); w1 (d x E*d_ff), expert
// e uses columns e*d_ff..; b1 (E*d_ff); w2 (E*d_ff x d), expert e uses rows
// e*d_ff..; b2 (d), shared.  pre / hidden / dpre are (T x d_ff) in expert-sorted
// row order: row i belongs to token perm[i].
#include "common.h"
#include "gemm.h"
#include <algorithm>

#include "moe.h"
#include "runtime.h"

using namespace asca;

static int moe_check(int T, int d, int d_ff, int E) {
    if (T < 0 || d <= 0 || d_ff <= 0 || E <= 0) return fail(ASCA_ERR_INVALID, "moe: bad shape T=%d d=%d d_ff=%d E=%d", T, d, d_ff, E);
    if ((long)E * d_ff > 0x7fffffffL) return fail(ASCA_ERR_INVALID, "moe: E*d_ff too large");
    return ASCA_OK;
}

// The two halves of the MoE backward: the data gradients on the critical path
// (dpre, dxn) and the weight / bias gradients that nothing later in the
// backward reads (dW1, db1, dW2, db2), so a caller may run them on another
// stream once dpre is written.
int asca::moe_bwd_data(const float* w1, const float* w2, const float* pre, const int32_t* perm,
                       const int32_t* offsets, const float* dout, int T, int d, int d_ff, int E, float* dxn,
                       float* dpre_ws, hipStream_t st) {
    if (T == 0) return ASCA_OK;
    // dpre = (dout[perm_e] @ w2[e]^T) * silu'(pre)
    GemmArgs dp = gemm_args();
    dp.A = dout;
    dp.lda = d;
    dp.a_rows = perm;
    dp.B = w2;
    dp.ldb = d;
    dp.b_gs = (long)d_ff * d;
    dp.C = dpre_ws;
    dp.ldc = d_ff;
    dp.aux = pre;
    dp.ld_aux = d_ff;
    dp.M = T;
    dp.N = d_ff;
    dp.K = d;
    dp.goff = offsets;
    dp.ngroups = E;
    dp.gmode = 1;
    int rc = gemm_launch(0, 1, EPI_SILU_BWD, dp, T, st, "moe_bwd_dpre");
    if (rc) return rc;
    // dxn[perm_e] = dpre_e @ w1[:, e]^T
    GemmArgs dx = gemm_args();
    dx.A = dpre_ws;
    dx.lda = d_ff;
    dx.B = w1;
    dx.ldb = (long)E * d_ff;
    dx.b_gs = d_ff;
    dx.C = dxn;
    dx.ldc = d;
    dx.c_rows = perm;
    dx.M = T;
    dx.N = d;
    dx.K = d_ff;
    dx.goff = offsets;
    dx.ngroups = E;
    dx.gmode = 1;
    return gemm_launch(0, 1, EPI_STORE, dx, T, st, "moe_bwd_dxn");
}

size_t asca::moe_bwd_weights_ws_floats(int T, int d, int d_ff, int E) {
    return std::max(colsum_ws_floats(T, d, false, 0), colsum_ws_floats(T, d_ff, true, E));
}

int asca::moe_bwd_weights(const float* xn, const float* hidden, const int32_t* perm, const int32_t* offsets,
                          const float* dout, const float* dpre_ws, int T, int d, int d_ff, int E, float* dw1,
                          float* db1, float* dw2, float* db2, int accumulate, Ws ws, hipStream_t st) {
    const float beta = accumulate ? 1.0f : 0.0f;
    // dW2[e] (+)= hidden_e^T dout[perm_e]
    GemmArgs g2 = gemm_args();
    g2.A = hidden;
    g2.lda = d_ff;
    g2.B = dout;
    g2.ldb = d;
    g2.b_rows = perm;
    g2.C = dw2;
    g2.ldc = d;
    g2.c_gs = (long)d_ff * d;
    g2.beta = beta;
    g2.M = d_ff;
    g2.N = d;
    g2.goff = offsets;
    g2.ngroups = E;
    g2.gmode = 2;
    int rc = gemm_launch(1, 0, EPI_STORE, g2, 0, st, "moe_bwd_dw2");
    if (rc) return rc;
    // db2 (+)= colsum(dout)
    if ((rc = colsum_launch(dout, T, d, d, nullptr, 0, db2, accumulate, ws, st))) return rc;
    // db1[e] (+)= colsum(dpre_e)
    if ((rc = colsum_launch(dpre_ws, T, d_ff, d_ff, offsets, E, db1, accumulate, ws, st))) return rc;
    // dW1[:, e] (+)= xn[perm_e]^T dpre_e
    GemmArgs g1 = gemm_args();
    g1.A = xn;
    g1.lda = d;
    g1.a_rows = perm;
    g1.B = dpre_ws;
    g1.ldb = d_ff;
    g1.C = dw1;
    g1.ldc = (long)E * d_ff;
    g1.c_gs = d_ff;
    g1.beta = beta;
    g1.M = d;
    g1.N = d_ff;
    g1.goff = offsets;
    g1.ngroups = E;
    g1.gmode = 2;
    return gemm_launch(1, 0, EPI_STORE, g1, 0, st, "moe_bwd_dw1");
}

extern "C" {

int asca_moe_fwd(const float* xn, const float* w1, const float* b1, const float* w2, const float* b2,
                 const int32_t* perm, const int32_t* offsets, int T, int d, int d_ff, int n_experts, float* out,
                 float* pre, float* hidden, void* stream) {
    int rc = moe_check(T, d, d_ff, n_experts);
    if (rc || T == 0) return rc;
    if (!xn || !w1 || !b1 || !w2 || !b2 || !perm || !offsets || !out || !pre || !hidden)
        return fail(ASCA_ERR_INVALID, "asca_moe_fwd: null pointer");
    const hipStream_t st = as_stream(stream);
    // pre = xn[perm] @ w1[:, e] + b1[e];  hidden = silu(pre)
    GemmArgs a = gemm_args();
    a.A = xn;
    a.lda = d;
    a.a_rows = perm;
    a.B = w1;
    a.ldb = (long)n_experts * d_ff;
    a.b_gs = d_ff;
    a.C = pre;
    a.ldc = d_ff;
    a.bias = b1;
    a.bias_gs = d_ff;
    a.aux_out = hidden;
    a.ld_aux = d_ff;
    a.M = T;
    a.N = d_ff;
    a.K = d;
    a.goff = offsets;
    a.ngroups = n_experts;
    a.gmode = 1;
    rc = gemm_launch(0, 0, EPI_SILU, a, T, st, "moe_fwd_w1");
    if (rc) return rc;
    // out[perm] = hidden @ w2[e] + b2
    GemmArgs b = gemm_args();
    b.A = hidden;
    b.lda = d_ff;
    b.B = w2;
    b.ldb = d;
    b.b_gs = (long)d_ff * d;
    b.C = out;
    b.ldc = d;
    b.c_rows = perm;
    b.bias = b2;
    b.M = T;
    b.N = d;
    b.K = d_ff;
    b.goff = offsets;
    b.ngroups = n_experts;
    b.gmode = 1;
    return gemm_launch(0, 0, EPI_STORE, b, T, st, "moe_fwd_w2");
}

int asca_moe_bwd(const float* xn, const float* w1, const float* w2, const float* pre, const float* hidden,
                 const int32_t* perm, const int32_t* offsets, const float* dout, int T, int d, int d_ff,
                 int n_experts, float* dxn, float* dw1, float* db1, float* dw2, float* db2, float* dpre_ws,
                 int accumulate, void* stream) {
    int rc = moe_check(T, d, d_ff, n_experts);
    if (rc) return rc;
    if (!xn || !w1 || !w2 || !pre || !hidden || !perm || !offsets || !dout || !dxn || !dw1 || !db1 || !dw2 ||
        !db2 || !dpre_ws)
        return fail(ASCA_ERR_INVALID, "asca_moe_bwd: null pointer");
    const hipStream_t st = as_stream(stream);
    if ((rc = moe_bwd_data(w1, w2, pre, perm, offsets, dout, T, d, d_ff, n_experts, dxn, dpre_ws, st))) return rc;
    // the column sums' partials: stream-ordered scratch (the reference's
    // moe_bwd_dev takes no workspace beyond dpre)
    StreamScratch sc;
    if ((rc = sc.get(moe_bwd_weights_ws_floats(T, d, d_ff, n_experts), st))) return rc;
    rc = moe_bwd_weights(xn, hidden, perm, offsets, dout, dpre_ws, T, d, d_ff, n_experts, dw1, db1, dw2, db2,
                         accumulate, sc.ws, st);
    const int rf = sc.release(st);
    return rc ? rc : rf;
}

}  // extern "C"
