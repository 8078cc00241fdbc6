// Internal interface of the MFMA GEMM (gemm.hip) for the composite operators
// (moe.hip, model.hip).  Not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>

#include "runtime.h"

namespace asca {

enum : int { EPI_STORE = 0, EPI_SILU = 1, EPI_SILU_BWD = 2 };

// One (possibly grouped, possibly split-K) GEMM:
//   C = alpha * op(A) op(B) (+ bias per column) (+ beta * C) (+ R)
// gmode 0: plain; gmode 1: M varies per group (rows goff[g]..goff[g+1] of the
// sorted row space); gmode 2: K varies per group; gmode 3: ngroups independent
// products of one shape, operand g at A + g*a_gs, B + g*b_gs, C + g*c_gs.  Row indirections map the
// operand's storage-row index (sorted space) to the stored row.
struct GemmArgs {
    const float* A;
    const float* B;
    float* C;
    long lda, ldb, ldc;
    int M, N, K;  // M (gmode 1) and K (gmode 2) come per group from goff
    float alpha, beta;
    const int* a_rows;  // storage-row indirection of A, B and C (or null)
    const int* b_rows;
    const int* c_rows;
    const float* bias;
    const float* resid;  // EPI_STORE: residual added per element (rows as C's, stride ld_resid), or null
    long ld_resid;
    long r_gs;           // per-group stride of resid
    const float* aux;  // EPI_SILU_BWD: pre (rows in group/sorted space)
    float* aux_out;    // EPI_SILU: hidden
    long ld_aux;
    const int* goff;  // group offsets [ngroups + 1]
    int ngroups, gmode;
    long a_gs, b_gs, c_gs, bias_gs;  // per-group pointer strides (elements)
    int tiles_m, tiles_n;
    long k_per_split;     // split-K: K range of blockIdx.y
    long c_split_stride;  // split-K: partial buffer stride per split
};

GemmArgs gemm_args();
// m_total: for gmode 1, the total rows over all groups (bounds the grid).
int gemm_launch(int ta, int tb, int epi, GemmArgs a, long m_total, hipStream_t st, const char* name);
// Skinny products with n <= 16 columns (the gate projection): Y (T x n, ld n)
// = X W + b, and G (K x n, ld n) = X^T D with db = column sums of D (db may be
// null).  Shapes the 16-wide kernels do not take go to the general GEMM.
int skinny_fwd_launch(const float* X, long ldx, const float* W, const float* b, float* Y, long T, int K, int n,
                      hipStream_t st);
int skinny_wgrad_launch(const float* X, long ldx, const float* D, float* G, float* db, long T, int K, int n,
                        Ws ws, hipStream_t st);
size_t skinny_wgrad_ws_floats(long T, int K, int n);
// out[g*N + c] (+)= column sums of X over the rows of group g (or all rows);
// ws holds the row-slice partials (colsum_ws_floats).
int colsum_launch(const float* X, long rows, int N, long ldx, const int* goff, int ngroups, float* out,
                  int accumulate, Ws ws, hipStream_t st);
size_t colsum_ws_floats(long rows, int N, bool grouped, int ngroups);
// Plain product C = alpha op(A) op(B) + beta C (+ bias per column), the
// arithmetic of asca_gemm; split-K partials go to ws (gemm_ws_floats of the
// shape; 0 when the product does not split).
int gemm_run(int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A, long lda, const float* B,
             long ldb, float beta, float* C, long ldc, const float* bias, Ws ws, hipStream_t st);
size_t gemm_ws_floats(int M, int N, int K);
int gemm_check(int trans_a, int trans_b, int M, int N, int K, const float* A, long lda, const float* B, long ldb,
               const float* C, long ldc);

}  // namespace asca
