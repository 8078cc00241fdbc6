// Chunked (WY/UT-transform) form of the gated delta rule, forward and
// backward, with every dense product on the MFMA GEMM (gemm.hip, batched over
// chunks).  The reference specifies this form without implementing it
// (docs/SPEC_V2.md:50-69); the math is that of the recurrence
// (rust/src/delta.rs:244-334, :421-613).
//
// Per chunk of C steps (gamma_t = prod_{m<=t} alpha_m, Gamma[t,i] = gamma_t/gamma_i
// for i <= t, computed as running products, never as 1/gamma):
//   A = K K^T, B = Q K^T, L = strict_tril(diag(beta)(Gamma o A)), T = (I + L)^-1,
//   M = tril(Gamma o B), Uv = T diag(beta) V, W = T diag(beta gamma) K,
//   Qp = diag(gamma) Q - M W, Kt = diag(Gamma[C-1, :]) K,
//   G' = gamma_C I - Kt^T W, H = Kt^T Uv,
// then per (sequence, head) over chunks S_{c+1} = G'_c S_c + H_c, and
// O_c = Qp S_c + M Uv.  The backward runs E_c = Qp^T dO_c and the reverse scan
// dS'_{c-1} = G'_c^T dS'_c + E_c (dS' = gradient of the state after a chunk),
// then per chunk (all independent):
//   U = Uv - W S, dU = M^T dO + Kt dS', dM = tril(dO U^T), dW = -dU S^T,
//   Y = T^T dU, Z = T^T dW, dKt = U dS'^T,
//   dL = -strict_tril(Y Uv^T + Z W^T), dA = dL o beta o Gamma,
//   dq = diag(gamma) dO S^T + (Gamma o dM) K,
//   dk = (Gamma o dM)^T Q + (dA + dA^T) K + diag(beta gamma) Z + diag(Gamma[C-1,:]) dKt,
//   dv = diag(beta) Y, and the scalar gradients of beta and alpha (through
//   gamma and Gamma, summed as d log alpha).
//
// Layout: inputs are token-major as everywhere in this library, q, k, v, dO as
// bf16 (raw 16-bit patterns, widened exactly to f32), gates f32.  The workspace
// holds unit-major f32 copies ([unit][t][dh], unit = b*H + h, T padded to a
// multiple of C with identity steps: q = k = v = 0, alpha = 1, beta = 0) and the
// per-chunk intermediates, so every batched product has one stride per chunk.
#include "common.h"
#include "gemm.h"
#include "runtime.h"

namespace asca {

struct ChunkDims {
    int B, T, H, dh, C, NC, Tp;
    long U, N, CD, CC, DD;
};

static ChunkDims chunk_dims(int B, int T, int H, int dh, int C) {
    ChunkDims d;
    d.B = B;
    d.T = T;
    d.H = H;
    d.dh = dh;
    d.C = C;
    d.NC = (T + C - 1) / C;
    d.Tp = d.NC * C;
    d.U = (long)B * H;
    d.N = d.U * d.NC;
    d.CD = (long)C * dh;
    d.CC = (long)C * C;
    d.DD = (long)dh * dh;
    return d;
}

// Workspace regions (floats).  Forward: persistent for the backward unless
// marked; backward regions follow.
struct ChunkWs {
    float *Qu, *Ku, *Vu, *al, *be, *gam, *gt, *gC, *Gam, *Am, *Bm, *Tm, *Mm, *Uv, *W, *Qp, *Kt, *Gp, *S;
    float *Vb, *Kbg, *Qg, *H, *Ou;  // forward temporaries
    float *dOu, *dOg, *E, *dSp, *Uu, *dU, *dMr, *dW, *Y, *Z, *dKt, *Pqs, *dLs, *GdM, *dAs, *dqu, *dku, *dal,
        *dbe;
    size_t total;  // floats
};

static ChunkWs chunk_ws(const ChunkDims& d, float* base) {
    ChunkWs w;
    size_t off = 0;
    auto take = [&](size_t n) {
        float* p = base ? base + off : nullptr;
        off += (n + 63) / 64 * 64;  // 256-byte aligned regions
        return p;
    };
    const size_t N = d.N, CD = d.CD, CC = d.CC, DD = d.DD, C = d.C;
    w.Qu = take(N * CD);
    w.Ku = take(N * CD);
    w.Vu = take(N * CD);
    w.al = take(N * C);
    w.be = take(N * C);
    w.gam = take(N * C);
    w.gt = take(N * C);
    w.gC = take(N);
    w.Gam = take(N * CC);
    w.Am = take(N * CC);
    w.Bm = take(N * CC);
    w.Tm = take(N * CC);
    w.Mm = take(N * CC);
    w.Uv = take(N * CD);
    w.W = take(N * CD);
    w.Qp = take(N * CD);
    w.Kt = take(N * CD);
    w.Gp = take(N * DD);
    w.S = take(N * DD);
    w.Vb = take(N * CD);
    w.Kbg = take(N * CD);
    w.Qg = take(N * CD);
    w.H = take(N * DD);
    w.Ou = take(N * CD);
    w.dOu = take(N * CD);
    w.dOg = take(N * CD);
    w.E = take(N * DD);
    w.dSp = take(N * DD);
    w.Uu = take(N * CD);
    w.dU = take(N * CD);
    w.dMr = take(N * CC);
    w.dW = take(N * CD);
    w.Y = take(N * CD);
    w.Z = take(N * CD);
    w.dKt = take(N * CD);
    w.Pqs = take(N * CD);
    w.dLs = take(N * CC);
    w.GdM = take(N * CC);
    w.dAs = take(N * CC);
    w.dqu = take(N * CD);
    w.dku = take(N * CD);
    w.dal = take(N * C);
    w.dbe = take(N * C);
    w.total = off;
    return w;
}

ASCA_DEV float bf16_to_f32(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }

// token-major bf16 (B*T, H*dh) -> unit-major f32 [u][Tp][dh], zero padding
__global__ __launch_bounds__(256) void ck_in_k(const uint16_t* __restrict__ src, float* __restrict__ dst, int T,
                                               int H, int dh, int Tp, long total) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int j = (int)(i % dh);
    const long r = i / dh;
    const int t = (int)(r % Tp);
    const long u = r / Tp;
    const long b = u / H, h = u % H;
    dst[i] = t < T ? bf16_to_f32(src[(b * T + t) * (long)H * dh + h * dh + j]) : 0.0f;
}

// gates (B*T, H) -> unit-major [u][Tp]; padding steps are identities (alpha 1, beta 0)
__global__ __launch_bounds__(256) void ck_gates_in_k(const float* __restrict__ alpha, const float* __restrict__ beta,
                                                     float* __restrict__ al, float* __restrict__ be, int T, int H,
                                                     int Tp, long total) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int t = (int)(i % Tp);
    const long u = i / Tp;
    const long b = u / H, h = u % H;
    const bool in = t < T;
    al[i] = in ? alpha[(b * T + t) * H + h] : 1.0f;
    be[i] = in ? beta[(b * T + t) * H + h] : 0.0f;
}

// Per chunk: gamma, Gamma, Gamma[C-1, :], gamma_C and the row-scaled copies
// Vb = beta V, Kbg = beta gamma K, Kt = Gamma[C-1,:] K, Qg = gamma Q.
__global__ __launch_bounds__(256) void ck_gamma_k(const float* __restrict__ al, const float* __restrict__ be,
                                                  const float* __restrict__ Qu, const float* __restrict__ Ku,
                                                  const float* __restrict__ Vu, int C, int dh,
                                                  float* __restrict__ gam, float* __restrict__ gt,
                                                  float* __restrict__ gC, float* __restrict__ Gam,
                                                  float* __restrict__ Vb, float* __restrict__ Kbg,
                                                  float* __restrict__ Kt, float* __restrict__ Qg) {
    __shared__ float a_s[64], b_s[64], g_s[64], gt_s[64];
    const long n = blockIdx.x;
    const int tid = threadIdx.x;
    if (tid < C) {
        a_s[tid] = al[n * C + tid];
        b_s[tid] = be[n * C + tid];
    }
    __syncthreads();
    if (tid == 0) {
        float g = 1.0f;
        for (int t = 0; t < C; ++t) {
            g *= a_s[t];
            g_s[t] = g;
        }
    }
    if (tid < C) {  // column i of Gamma by running products down the column
        const int i = tid;
        float* G = Gam + n * C * C;
        float v = 1.0f;
        for (int t = 0; t < C; ++t) {
            if (t > i) v *= a_s[t];
            G[t * C + i] = t >= i ? v : 0.0f;
        }
        gt_s[i] = v;  // Gamma[C-1, i]
    }
    __syncthreads();
    if (tid < C) {
        gam[n * C + tid] = g_s[tid];
        gt[n * C + tid] = gt_s[tid];
    }
    if (tid == 0) gC[n] = g_s[C - 1];
    const long base = n * C * dh;
    for (int e = tid; e < C * dh; e += 256) {
        const int t = e / dh;
        const float q = Qu[base + e], k = Ku[base + e], v = Vu[base + e];
        Vb[base + e] = b_s[t] * v;
        Kbg[base + e] = (b_s[t] * g_s[t]) * k;
        Kt[base + e] = gt_s[t] * k;
        Qg[base + e] = g_s[t] * q;
    }
}

// Per chunk (one wave, thread = column): L from A, Gamma, beta; T = (I + L)^-1
// by forward substitution down each column; M = tril(Gamma o B).
__global__ __launch_bounds__(64) void ck_tri_k(const float* __restrict__ Am, const float* __restrict__ Bm,
                                               const float* __restrict__ Gam, const float* __restrict__ be, int C,
                                               float* __restrict__ Tm, float* __restrict__ Mm) {
    __shared__ float L[64][65];
    __shared__ float Tc[64][65];
    const long n = blockIdx.x;
    const int m = threadIdx.x;
    const float* A = Am + n * C * C;
    const float* Bq = Bm + n * C * C;
    const float* G = Gam + n * C * C;
    if (m < C) {
        for (int j = 0; j < C; ++j) {
            const float g = G[j * C + m];
            L[j][m] = m < j ? be[n * C + j] * (g * A[j * C + m]) : 0.0f;
            Mm[n * C * C + j * C + m] = m <= j ? g * Bq[j * C + m] : 0.0f;
        }
    }
    __syncthreads();
    if (m < C) {
        for (int j = 0; j < C; ++j) {
            float t;
            if (j < m) {
                t = 0.0f;
            } else if (j == m) {
                t = 1.0f;
            } else {
                float s = 0.0f;
                for (int i = m; i < j; ++i) s += L[j][i] * Tc[i][m];
                t = -s;
            }
            Tc[j][m] = t;
            Tm[n * C * C + j * C + m] = t;
        }
    }
}

// G'[n] += gamma_C[n] I  (the GEMM wrote -Kt^T W)
__global__ __launch_bounds__(256) void ck_diag_k(float* __restrict__ Gp, const float* __restrict__ gC, int dh,
                                                 long total) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const long n = i / dh;
    const int j = (int)(i % dh);
    Gp[n * (long)dh * dh + (long)j * dh + j] += gC[n];
}

// unit-major [u][Tp][w] -> token-major (B*T, H*w), dropping the padding
__global__ __launch_bounds__(256) void ck_out_k(const float* __restrict__ src, float* __restrict__ dst, int T, int H,
                                                int w, int Tp, long total) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;  // over token-major elements
    if (i >= total) return;
    const int col = (int)(i % ((long)H * w));
    const long row = i / ((long)H * w);
    const long b = row / T;
    const int t = (int)(row % T);
    const int h = col / w, j = col % w;
    dst[i] = src[((b * H + h) * Tp + t) * (long)w + j];
}

// rows scaled: out[n][t][:] = s[n*C + t] * in[n][t][:]
__global__ __launch_bounds__(256) void ck_rowscale_k(const float* __restrict__ in, const float* __restrict__ s,
                                                     float* __restrict__ out, int dh, long total) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    out[i] = s[i / dh] * in[i];
}

// Per chunk: the C x C gradient terms and the scalar gradients.
//   GdM = Gamma o tril(dMr);  dL = -strict_tril(dLs);  dA = dL o beta_j o Gamma;
//   dAs = dA + dA^T;  dbeta_j = Y_j.V_j + gamma_j Z_j.K_j + sum_i dL Gamma A;
//   dgamma_t = beta_t Z_t.K_t + dO_t.(QS)_t (+ <dS', S> at t = C-1);
//   dGamma = dMr o B (tril) + dL beta A (+ K_i.dKt_i on row C-1);
//   dalpha_m = (sum_{t>=m} dgamma_t gamma_t + sum_{t>=m>i} dGamma Gamma) / alpha_m.
__global__ __launch_bounds__(256) void ck_bwd_scalars_k(
    const float* __restrict__ dMr, const float* __restrict__ dLs, const float* __restrict__ Gam,
    const float* __restrict__ Am, const float* __restrict__ Bm, const float* __restrict__ al,
    const float* __restrict__ be, const float* __restrict__ gam, const float* __restrict__ Y,
    const float* __restrict__ Vu, const float* __restrict__ Z, const float* __restrict__ Ku,
    const float* __restrict__ dOu, const float* __restrict__ Pqs, const float* __restrict__ dKt,
    const float* __restrict__ dSp, const float* __restrict__ S, int C, int dh, float* __restrict__ GdM,
    float* __restrict__ dAs, float* __restrict__ dal, float* __restrict__ dbe) {
    __shared__ float yv[64], zk[64], op[64], kk[64], dg[64], red[4];
    __shared__ float R[64][65];
    __shared__ float dAl[64][65];
    const long n = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const long cd = n * C * dh, cc = n * C * C;
    // row dots
    for (int t = w; t < C; t += 4) {
        float a = 0.f, b = 0.f, c = 0.f, e = 0.f;
        for (int j = lane; j < dh; j += 64) {
            const long o = cd + (long)t * dh + j;
            a += Y[o] * Vu[o];
            b += Z[o] * Ku[o];
            c += dOu[o] * Pqs[o];
            e += Ku[o] * dKt[o];
        }
        a = wave_sum(a);
        b = wave_sum(b);
        c = wave_sum(c);
        e = wave_sum(e);
        if (lane == 0) {
            yv[t] = a;
            zk[t] = b;
            op[t] = c;
            kk[t] = e;
        }
    }
    // <dS', S>
    float f = 0.0f;
    const long dd = (long)dh * dh;
    for (long e = tid; e < dd; e += 256) f += dSp[n * dd + e] * S[n * dd + e];
    f = wave_sum(f);
    if (lane == 0) red[w] = f;
    __syncthreads();
    const float fro = (red[0] + red[1]) + (red[2] + red[3]);
    // C x C terms: thread = column i (first C threads), rows j
    if (tid < C) {
        const int i = tid;
        for (int j = 0; j < C; ++j) {
            const long o = cc + (long)j * C + i;
            const float g = Gam[o], dm = i <= j ? dMr[o] : 0.0f;
            const float dl = i < j ? -dLs[o] : 0.0f;
            const float bj = be[n * C + j];
            GdM[o] = g * dm;
            dAl[j][i] = dl * bj * g;
            float dG = dm * Bm[o] + dl * bj * Am[o];
            if (j == C - 1) dG += kk[i];
            R[j][i] = i < j ? dG * g : 0.0f;
        }
    }
    __syncthreads();
    if (tid < C) {
        const int j = tid;
        // dA + dA^T, row j
        for (int i = 0; i < C; ++i) dAs[cc + (long)j * C + i] = dAl[j][i] + dAl[i][j];
        // dbeta_j
        float s = 0.0f;
        for (int i = 0; i < j; ++i) s += (-dLs[cc + (long)j * C + i]) * Gam[cc + (long)j * C + i] * Am[cc + (long)j * C + i];
        const float gj = gam[n * C + j];
        dbe[n * C + j] = yv[j] + gj * zk[j] + s;
        float dgam = be[n * C + j] * zk[j] + op[j];
        if (j == C - 1) dgam += fro;
        dg[j] = dgam * gj;
    }
    __syncthreads();
    if (tid < C) {
        const int m = tid;
        float s = 0.0f;
        for (int t = m; t < C; ++t) {
            s += dg[t];
            for (int i = 0; i < m; ++i) s += R[t][i];
        }
        dal[n * C + m] = s / al[n * C + m];
    }
}

// dk = dku + beta gamma Z + Gamma[C-1,:] dKt; dv = beta Y (unit-major -> token-major)
__global__ __launch_bounds__(256) void ck_bwd_out_k(const float* __restrict__ dqu, const float* __restrict__ dku,
                                                    const float* __restrict__ Z, const float* __restrict__ dKt,
                                                    const float* __restrict__ Y, const float* __restrict__ be,
                                                    const float* __restrict__ gam, const float* __restrict__ gt,
                                                    int T, int H, int dh, int Tp, float* __restrict__ dq,
                                                    float* __restrict__ dk, float* __restrict__ dv, long total) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int col = (int)(i % ((long)H * dh));
    const long row = i / ((long)H * dh);
    const long b = row / T;
    const int t = (int)(row % T);
    const int h = col / dh, j = col % dh;
    const long r = (b * H + h) * Tp + t;  // unit-major row
    const long o = r * dh + j;
    dq[i] = dqu[o];
    dk[i] = dku[o] + (be[r] * gam[r]) * Z[o] + gt[r] * dKt[o];
    dv[i] = be[r] * Y[o];
}

__global__ __launch_bounds__(256) void ck_gates_out_k(const float* __restrict__ dal, const float* __restrict__ dbe,
                                                      int T, int H, int Tp, float* __restrict__ da,
                                                      float* __restrict__ db, long total) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int h = (int)(i % H);
    const long row = i / H;
    const long b = row / T;
    const int t = (int)(row % T);
    const long r = (b * H + h) * Tp + t;
    da[i] = dal[r];
    db[i] = dbe[r];
}

// zero one d x d slot per unit: base[u * us + off + e], e < dd
__global__ __launch_bounds__(256) void ck_zero_slot_k(float* __restrict__ base, long us, long off, long dd,
                                                      long total) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    base[(i / dd) * us + off + (i % dd)] = 0.0f;
}

static unsigned nblk(long total) { return (unsigned)((total + 255) / 256); }

// batched product: ngroups independent (M x N) = op(A) op(B) with per-group strides
static int bgemm(int ta, int tb, int M, int N, int K, float alpha, const float* A, long lda, long a_gs,
                 const float* B, long ldb, long b_gs, float beta, float* C, long ldc, long c_gs, const float* R,
                 long r_gs, long groups, hipStream_t st, const char* name) {
    GemmArgs a = gemm_args();
    a.A = A;
    a.lda = lda;
    a.a_gs = a_gs;
    a.B = B;
    a.ldb = ldb;
    a.b_gs = b_gs;
    a.C = C;
    a.ldc = ldc;
    a.c_gs = c_gs;
    a.alpha = alpha;
    a.beta = beta;
    a.resid = R;
    a.ld_resid = ldc;
    a.r_gs = r_gs;
    a.M = M;
    a.N = N;
    a.K = K;
    a.ngroups = (int)groups;
    a.gmode = 3;
    return gemm_launch(ta, tb, EPI_STORE, a, 0, st, name);
}

static int chunk_check(int B, int T, int H, int dh, int C) {
    if (B < 0 || T < 0 || H < 0) return fail(ASCA_ERR_INVALID, "chunked: negative shape");
    if (C < 1 || C > 64) return fail(ASCA_ERR_UNSUPPORTED, "chunked: chunk %d outside 1..64", C);
    if (dh < 4 || dh > 256 || dh % 4) return fail(ASCA_ERR_UNSUPPORTED, "chunked: dh=%d (multiple of 4, 4..256)", dh);
    return ASCA_OK;
}

#define CK_LAUNCH(name, kern, grid, block, ...)                   \
    do {                                                          \
        int rc_ = pre_launch(name);                               \
        if (rc_) return rc_;                                      \
        hipLaunchKernelGGL(kern, grid, block, 0, st, __VA_ARGS__); \
        rc_ = post_launch(name);                                  \
        if (rc_) return rc_;                                      \
    } while (0)

}  // namespace asca

using namespace asca;

extern "C" {

int asca_chunk_ws_bytes(int B, int T, int H, int dh, int C, size_t* bytes) {
    if (!bytes) return fail(ASCA_ERR_INVALID, "null output pointer");
    int rc = chunk_check(B, T, H, dh, C);
    if (rc) return rc;
    *bytes = chunk_ws(chunk_dims(B, T, H, dh, C), nullptr).total * sizeof(float);
    return ASCA_OK;
}

int asca_chunk_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* alpha, const float* beta,
                   float* o, void* ws, int B, int T, int H, int dh, int C, void* stream) {
    int rc = chunk_check(B, T, H, dh, C);
    if (rc) return rc;
    if ((long)B * T * H == 0) return ASCA_OK;
    if (!q || !k || !v || !alpha || !beta || !o || !ws) return fail(ASCA_ERR_INVALID, "asca_chunk_fwd: null pointer");
    const ChunkDims d = chunk_dims(B, T, H, dh, C);
    const ChunkWs w = chunk_ws(d, reinterpret_cast<float*>(ws));
    const hipStream_t st = as_stream(stream);
    const long tot_in = d.U * d.Tp * dh;
    CK_LAUNCH("chunk_in", ck_in_k, dim3(nblk(tot_in)), dim3(256), q, w.Qu, T, H, dh, d.Tp, tot_in);
    CK_LAUNCH("chunk_in", ck_in_k, dim3(nblk(tot_in)), dim3(256), k, w.Ku, T, H, dh, d.Tp, tot_in);
    CK_LAUNCH("chunk_in", ck_in_k, dim3(nblk(tot_in)), dim3(256), v, w.Vu, T, H, dh, d.Tp, tot_in);
    CK_LAUNCH("chunk_gates_in", ck_gates_in_k, dim3(nblk(d.U * d.Tp)), dim3(256), alpha, beta, w.al, w.be, T, H, d.Tp,
              d.U * d.Tp);
    // per-chunk state-independent parts
    if ((rc = bgemm(0, 1, C, C, dh, 1.f, w.Ku, dh, d.CD, w.Ku, dh, d.CD, 0.f, w.Am, C, d.CC, nullptr, 0, d.N, st,
                    "chunk_KKt")))
        return rc;
    if ((rc = bgemm(0, 1, C, C, dh, 1.f, w.Qu, dh, d.CD, w.Ku, dh, d.CD, 0.f, w.Bm, C, d.CC, nullptr, 0, d.N, st,
                    "chunk_QKt")))
        return rc;
    CK_LAUNCH("chunk_gamma", ck_gamma_k, dim3((unsigned)d.N), dim3(256), w.al, w.be, w.Qu, w.Ku, w.Vu, C, dh, w.gam,
              w.gt, w.gC, w.Gam, w.Vb, w.Kbg, w.Kt, w.Qg);
    CK_LAUNCH("chunk_tri", ck_tri_k, dim3((unsigned)d.N), dim3(64), w.Am, w.Bm, w.Gam, w.be, C, w.Tm, w.Mm);
    if ((rc = bgemm(0, 0, C, dh, C, 1.f, w.Tm, C, d.CC, w.Vb, dh, d.CD, 0.f, w.Uv, dh, d.CD, nullptr, 0, d.N, st,
                    "chunk_Uv")) ||
        (rc = bgemm(0, 0, C, dh, C, 1.f, w.Tm, C, d.CC, w.Kbg, dh, d.CD, 0.f, w.W, dh, d.CD, nullptr, 0, d.N, st,
                    "chunk_W")) ||
        (rc = bgemm(0, 0, C, dh, C, -1.f, w.Mm, C, d.CC, w.W, dh, d.CD, 0.f, w.Qp, dh, d.CD, w.Qg, d.CD, d.N, st,
                    "chunk_Qp")) ||
        (rc = bgemm(1, 0, dh, dh, C, -1.f, w.Kt, dh, d.CD, w.W, dh, d.CD, 0.f, w.Gp, dh, d.DD, nullptr, 0, d.N, st,
                    "chunk_G")) ||
        (rc = bgemm(1, 0, dh, dh, C, 1.f, w.Kt, dh, d.CD, w.Uv, dh, d.CD, 0.f, w.H, dh, d.DD, nullptr, 0, d.N, st,
                    "chunk_H")))
        return rc;
    CK_LAUNCH("chunk_diag", ck_diag_k, dim3(nblk(d.N * dh)), dim3(256), w.Gp, w.gC, dh, d.N * dh);
    // state scan over chunks: S_0 = 0, S_{c+1} = G'_c S_c + H_c
    const long us = (long)d.NC * d.DD;  // per-unit stride of per-chunk d x d blocks
    CK_LAUNCH("chunk_zero", ck_zero_slot_k, dim3(nblk(d.U * d.DD)), dim3(256), w.S, us, 0L, d.DD, d.U * d.DD);
    for (int c = 0; c + 1 < d.NC; ++c) {
        const long oc = (long)c * d.DD;
        if ((rc = bgemm(0, 0, dh, dh, dh, 1.f, w.Gp + oc, dh, us, w.S + oc, dh, us, 0.f, w.S + oc + d.DD, dh, us,
                        w.H + oc, us, d.U, st, "chunk_scan")))
            return rc;
    }
    // outputs: O = Qp S + M Uv
    if ((rc = bgemm(0, 0, C, dh, dh, 1.f, w.Qp, dh, d.CD, w.S, dh, d.DD, 0.f, w.Ou, dh, d.CD, nullptr, 0, d.N, st,
                    "chunk_O1")) ||
        (rc = bgemm(0, 0, C, dh, C, 1.f, w.Mm, C, d.CC, w.Uv, dh, d.CD, 1.f, w.Ou, dh, d.CD, nullptr, 0, d.N, st,
                    "chunk_O2")))
        return rc;
    const long tot_out = (long)B * T * H * dh;
    CK_LAUNCH("chunk_out", ck_out_k, dim3(nblk(tot_out)), dim3(256), w.Ou, o, T, H, dh, d.Tp, tot_out);
    return ASCA_OK;
}

int asca_chunk_bwd(const uint16_t* d_o, void* ws, float* dq, float* dk, float* dv, float* dalpha, float* dbeta, int B,
                   int T, int H, int dh, int C, void* stream) {
    int rc = chunk_check(B, T, H, dh, C);
    if (rc) return rc;
    if ((long)B * T * H == 0) return ASCA_OK;
    if (!d_o || !ws || !dq || !dk || !dv || !dalpha || !dbeta)
        return fail(ASCA_ERR_INVALID, "asca_chunk_bwd: null pointer");
    const ChunkDims d = chunk_dims(B, T, H, dh, C);
    const ChunkWs w = chunk_ws(d, reinterpret_cast<float*>(ws));
    const hipStream_t st = as_stream(stream);
    const long tot_in = d.U * d.Tp * dh;
    CK_LAUNCH("chunk_in", ck_in_k, dim3(nblk(tot_in)), dim3(256), d_o, w.dOu, T, H, dh, d.Tp, tot_in);
    CK_LAUNCH("chunk_rowscale", ck_rowscale_k, dim3(nblk(tot_in)), dim3(256), w.dOu, w.gam, w.dOg, dh, tot_in);
    // E_c = Qp^T dO_c; reverse scan dS'_{c-1} = G'_c^T dS'_c + E_c, dS'_{NC-1} = 0
    if ((rc = bgemm(1, 0, dh, dh, C, 1.f, w.Qp, dh, d.CD, w.dOu, dh, d.CD, 0.f, w.E, dh, d.DD, nullptr, 0, d.N, st,
                    "chunk_E")))
        return rc;
    const long us = (long)d.NC * d.DD;
    CK_LAUNCH("chunk_zero", ck_zero_slot_k, dim3(nblk(d.U * d.DD)), dim3(256), w.dSp, us, (long)(d.NC - 1) * d.DD,
              d.DD, d.U * d.DD);
    for (int c = d.NC - 1; c >= 1; --c) {
        const long oc = (long)c * d.DD;
        if ((rc = bgemm(1, 0, dh, dh, dh, 1.f, w.Gp + oc, dh, us, w.dSp + oc, dh, us, 0.f, w.dSp + oc - d.DD, dh, us,
                        w.E + oc, us, d.U, st, "chunk_scan_bwd")))
            return rc;
    }
    // per-chunk gradients
    const long N = d.N, CD = d.CD, CC = d.CC, DD = d.DD;
    if ((rc = bgemm(0, 0, C, dh, dh, -1.f, w.W, dh, CD, w.S, dh, DD, 0.f, w.Uu, dh, CD, w.Uv, CD, N, st, "chunk_U")) ||
        (rc = bgemm(1, 0, C, dh, C, 1.f, w.Mm, C, CC, w.dOu, dh, CD, 0.f, w.dU, dh, CD, nullptr, 0, N, st,
                    "chunk_dU1")) ||
        (rc = bgemm(0, 0, C, dh, dh, 1.f, w.Kt, dh, CD, w.dSp, dh, DD, 1.f, w.dU, dh, CD, nullptr, 0, N, st,
                    "chunk_dU2")) ||
        (rc = bgemm(0, 1, C, C, dh, 1.f, w.dOu, dh, CD, w.Uu, dh, CD, 0.f, w.dMr, C, CC, nullptr, 0, N, st,
                    "chunk_dM")) ||
        (rc = bgemm(0, 1, C, dh, dh, -1.f, w.dU, dh, CD, w.S, dh, DD, 0.f, w.dW, dh, CD, nullptr, 0, N, st,
                    "chunk_dW")) ||
        (rc = bgemm(1, 0, C, dh, C, 1.f, w.Tm, C, CC, w.dU, dh, CD, 0.f, w.Y, dh, CD, nullptr, 0, N, st,
                    "chunk_Y")) ||
        (rc = bgemm(1, 0, C, dh, C, 1.f, w.Tm, C, CC, w.dW, dh, CD, 0.f, w.Z, dh, CD, nullptr, 0, N, st,
                    "chunk_Z")) ||
        (rc = bgemm(0, 1, C, dh, dh, 1.f, w.Uu, dh, CD, w.dSp, dh, DD, 0.f, w.dKt, dh, CD, nullptr, 0, N, st,
                    "chunk_dKt")) ||
        (rc = bgemm(0, 0, C, dh, dh, 1.f, w.Qu, dh, CD, w.S, dh, DD, 0.f, w.Pqs, dh, CD, nullptr, 0, N, st,
                    "chunk_QS")) ||
        (rc = bgemm(0, 1, C, C, dh, 1.f, w.Y, dh, CD, w.Uv, dh, CD, 0.f, w.dLs, C, CC, nullptr, 0, N, st,
                    "chunk_dL1")) ||
        (rc = bgemm(0, 1, C, C, dh, 1.f, w.Z, dh, CD, w.W, dh, CD, 1.f, w.dLs, C, CC, nullptr, 0, N, st,
                    "chunk_dL2")))
        return rc;
    CK_LAUNCH("chunk_bwd_scalars", ck_bwd_scalars_k, dim3((unsigned)N), dim3(256), w.dMr, w.dLs, w.Gam, w.Am, w.Bm,
              w.al, w.be, w.gam, w.Y, w.Vu, w.Z, w.Ku, w.dOu, w.Pqs, w.dKt, w.dSp, w.S, C, dh, w.GdM, w.dAs, w.dal,
              w.dbe);
    if ((rc = bgemm(0, 1, C, dh, dh, 1.f, w.dOg, dh, CD, w.S, dh, DD, 0.f, w.dqu, dh, CD, nullptr, 0, N, st,
                    "chunk_dq1")) ||
        (rc = bgemm(0, 0, C, dh, C, 1.f, w.GdM, C, CC, w.Ku, dh, CD, 1.f, w.dqu, dh, CD, nullptr, 0, N, st,
                    "chunk_dq2")) ||
        (rc = bgemm(1, 0, C, dh, C, 1.f, w.GdM, C, CC, w.Qu, dh, CD, 0.f, w.dku, dh, CD, nullptr, 0, N, st,
                    "chunk_dk1")) ||
        (rc = bgemm(0, 0, C, dh, C, 1.f, w.dAs, C, CC, w.Ku, dh, CD, 1.f, w.dku, dh, CD, nullptr, 0, N, st,
                    "chunk_dk2")))
        return rc;
    const long tot_out = (long)B * T * H * dh;
    CK_LAUNCH("chunk_bwd_out", ck_bwd_out_k, dim3(nblk(tot_out)), dim3(256), w.dqu, w.dku, w.Z, w.dKt, w.Y, w.be,
              w.gam, w.gt, T, H, dh, d.Tp, dq, dk, dv, tot_out);
    const long tot_g = (long)B * T * H;
    CK_LAUNCH("chunk_gates_out", ck_gates_out_k, dim3(nblk(tot_g)), dim3(256), w.dal, w.dbe, T, H, d.Tp, dalpha, dbeta,
              tot_g);
    return ASCA_OK;
}

}  // extern "C"
