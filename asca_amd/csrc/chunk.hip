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

// fusedlayout: the C = 64, dh = 128 bf16 kernels' workspace (see below); the
// f32 entry points always take the decomposed layout.
static ChunkWs chunk_ws(const ChunkDims& d, float* base, bool fusedlayout = true) {
    ChunkWs w;
    size_t off = 0;
    auto take = [&](size_t n) {
        float* p = base ? base + off : nullptr;
        off += (n + 63) / 64 * 64;  // 256-byte aligned regions
        return p;
    };
    const size_t N = d.N, CD = d.CD, CC = d.CC, DD = d.DD, C = d.C;
    // the fused C = 64, dh = 128 kernels need only the forward factors, the
    // states and U; the decomposed path's other regions are left out
    const bool fused = fusedlayout && d.C == 64 && d.dh == 128;
    auto opt = [&](size_t n) -> float* { return fused ? nullptr : take(n); };
    // f32 copies of q, k, v: the fused kernels read the bf16 inputs instead
    w.Qu = opt(N * CD);
    w.Ku = opt(N * CD);
    w.Vu = opt(N * CD);
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
    w.Kt = opt(N * CD);
    w.Gp = opt(N * DD);
    w.S = take(N * DD);
    w.Vb = opt(N * CD);
    w.Kbg = opt(N * CD);
    w.Qg = opt(N * CD);
    w.H = opt(N * DD);
    w.Ou = opt(N * CD);
    w.dOu = opt(N * CD);
    w.dOg = opt(N * CD);
    w.E = opt(N * DD);
    w.dSp = take(N * DD);
    w.Uu = take(N * CD);
    w.dU = opt(N * CD);
    w.dMr = opt(N * CC);
    w.dW = opt(N * CD);
    w.Y = opt(N * CD);
    w.Z = opt(N * CD);
    w.dKt = opt(N * CD);
    w.Pqs = opt(N * CD);
    w.dLs = opt(N * CC);
    w.GdM = opt(N * CC);
    w.dAs = opt(N * CC);
    w.dqu = opt(N * CD);
    w.dku = opt(N * CD);
    w.dal = opt(N * C);
    w.dbe = opt(N * C);
    w.total = off;
    return w;
}

ASCA_DEV float bf16_to_f32(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }

// token-major bf16 (B*T, H*dh) -> unit-major f32 [u][Tp][dh], zero padding;
// four elements per thread (dh % 4 == 0), 32-bit indices (sizes checked)
__global__ __launch_bounds__(256) void ck_in_k(const uint16_t* __restrict__ src, float* __restrict__ dst, int T,
                                               int H, int dh, int Tp, int total4) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= total4) return;
    const int q4 = dh >> 2;
    const int j = 4 * (i % q4);
    const int r = i / q4;
    const int t = r % Tp, u = r / Tp;
    const int b = u / H, h = u - b * H;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < T) {
        const uint2 x = *reinterpret_cast<const uint2*>(src + ((size_t)(b * T + t) * H + h) * dh + j);
        v = make_float4(__uint_as_float(x.x << 16), __uint_as_float(x.x & 0xffff0000u), __uint_as_float(x.y << 16),
                        __uint_as_float(x.y & 0xffff0000u));
    }
    reinterpret_cast<float4*>(dst)[i] = v;
}

// token-major f32 (B*T, H*dh) -> unit-major f32 [u][Tp][dh], zero padding;
// four elements per thread, one 16-byte access when the source is 16-byte
// aligned (AL)
template <bool AL>
__global__ __launch_bounds__(256) void ck_in_f32_k(const float* __restrict__ src, float* __restrict__ dst, int T,
                                                   int H, int dh, int Tp, int total4) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= total4) return;
    const int q4 = dh >> 2;
    const int j = 4 * (i % q4);
    const int r = i / q4;
    const int t = r % Tp, u = r / Tp;
    const int b = u / H, h = u - b * H;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < T) {
        const float* const x = src + ((size_t)(b * T + t) * H + h) * dh + j;
        if constexpr (AL) v = *reinterpret_cast<const float4*>(x);
        else v = make_float4(x[0], x[1], x[2], x[3]);
    }
    reinterpret_cast<float4*>(dst)[i] = v;
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

// Per chunk: L from A, Gamma, beta (all 256 threads, four rows at a time);
// T = (I + L)^-1 by forward substitution down each column (thread = column);
// M = tril(Gamma o B).
__global__ __launch_bounds__(256) void ck_tri_k(const float* __restrict__ Am, const float* __restrict__ Bm,
                                                const float* __restrict__ Gam, const float* __restrict__ be, int C,
                                                float* __restrict__ Tm, float* __restrict__ Mm) {
    __shared__ float L[64][65];
    __shared__ float Tc[64][65];
    const long n = blockIdx.x;
    const int tid = threadIdx.x, m = tid & 63, r4 = tid >> 6;
    const long cc = n * C * C;
    if (m < C) {
        for (int j = r4; j < C; j += 4) {
            const long o = cc + (long)j * C + m;
            const float g = Gam[o];
            L[j][m] = m < j ? be[n * C + j] * (g * Am[o]) : 0.0f;
            Mm[o] = m <= j ? g * Bm[o] : 0.0f;
        }
    }
    __syncthreads();
    if (tid < C) {
        for (int j = 0; j < C; ++j) {
            float t;
            if (j < m) {
                t = 0.0f;
            } else if (j == m) {
                t = 1.0f;
            } else {
                float s0 = 0.0f, s1 = 0.0f;
                int i = m;
                for (; i + 1 < j; i += 2) {
                    s0 += L[j][i] * Tc[i][m];
                    s1 += L[j][i + 1] * Tc[i + 1][m];
                }
                if (i < j) s0 += L[j][i] * Tc[i][m];
                t = -(s0 + s1);
            }
            Tc[j][m] = t;
        }
    }
    __syncthreads();
    if (m < C)
        for (int j = r4; j < C; j += 4) Tm[cc + (long)j * C + m] = Tc[j][m];
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

// unit-major [u][Tp][w] -> token-major (B*T, H*w), dropping the padding (w % 4 == 0)
__global__ __launch_bounds__(256) void ck_out_k(const float* __restrict__ src, float* __restrict__ dst, int T, int H,
                                                int w, int Tp, int total4) {
    const int i = blockIdx.x * 256 + threadIdx.x;  // float4 index over token-major elements
    if (i >= total4) return;
    const int hw4 = (H * w) >> 2;
    const int col = 4 * (i % hw4);
    const int row = i / hw4;
    const int b = row / T, t = row - b * T;
    const int h = col / w, j = col - h * w;
    reinterpret_cast<float4*>(dst)[i] =
        *reinterpret_cast<const float4*>(src + ((size_t)(b * H + h) * Tp + t) * w + j);
}

// rows scaled: out[n][t][:] = s[n*C + t] * in[n][t][:]  (dh % 4 == 0)
__global__ __launch_bounds__(256) void ck_rowscale_k(const float* __restrict__ in, const float* __restrict__ s,
                                                     float* __restrict__ out, int dh, int total4) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= total4) return;
    const float f = s[i / (dh >> 2)];
    float4 v = reinterpret_cast<const float4*>(in)[i];
    v.x *= f;
    v.y *= f;
    v.z *= f;
    v.w *= f;
    reinterpret_cast<float4*>(out)[i] = v;
}

// Per chunk: the C x C gradient terms and the scalar gradients.
//   GdM = Gamma o tril(dMr);  dL = -strict_tril(dLs);  dA = dL o beta_j o Gamma;
//   dAs = dA + dA^T;  dbeta_j = Y_j.V_j + gamma_j Z_j.K_j + sum_i dL Gamma A;
//   dgamma_t = beta_t Z_t.K_t + dO_t.(QS)_t (+ <dS', S> at t = C-1);
//   dGamma = dMr o B (tril) + dL beta A (+ K_i.dKt_i on row C-1);
//   dalpha_m = gamma_{m-1} s(m) + sum_{t>=m} Gamma[t][m] c_t(m), the derivative
//   of every running product with alpha_m left out (no division: exact for
//   alpha_m = 0), where s(m) = sum_{t>=m} Gamma[t][m] dgamma_t and
//   c_t(m) = sum_{i<m} dGamma[t][i] Gamma[m-1][i], i.e. c_t(0) = 0,
//   c_t(m+1) = alpha_m c_t(m) + dGamma[t][m].
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
    __shared__ float Pb[64][65];
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
    // C x C terms, four rows at a time: thread (i = tid & 63, rows j = tid >> 6 + 4k)
    {
        const int i = tid & 63;
        if (i < C) {
            for (int j = tid >> 6; j < C; j += 4) {
                const long o = cc + (long)j * C + i;
                const float g = Gam[o], dm = i <= j ? dMr[o] : 0.0f;
                const float dl = i < j ? -dLs[o] : 0.0f;
                const float bj = be[n * C + j], a = Am[o];
                GdM[o] = g * dm;
                dAl[j][i] = dl * bj * g;
                float dG = dm * Bm[o] + dl * bj * a;
                if (j == C - 1) dG += kk[i];
                R[j][i] = i < j ? dG : 0.0f;   // dGamma, strictly lower
                Pb[j][i] = dl * g * a;  // dbeta row terms
            }
        }
    }
    __syncthreads();
    {
        const int i = tid & 63;
        if (i < C)
            for (int j = tid >> 6; j < C; j += 4) dAs[cc + (long)j * C + i] = dAl[j][i] + dAl[i][j];
    }
    if (tid < C) {
        const int j = tid;
        float s = 0.0f;
        for (int i = 0; i < j; ++i) s += Pb[j][i];
        const float gj = gam[n * C + j];
        dbe[n * C + j] = yv[j] + gj * zk[j] + s;
        float dgam = be[n * C + j] * zk[j] + op[j];
        if (j == C - 1) dgam += fro;
        dg[j] = dgam;
    }
    __syncthreads();
    // dAl is free again: row t of X[t][m] = Gamma[t][m] c_t(m), one thread per row
    if (tid < C) {
        const int t = tid;
        float cm = 0.0f;   // c_t(m)
        for (int m = 0; m < C; ++m) {
            dAl[t][m] = m <= t ? Gam[cc + (long)t * C + m] * cm : 0.0f;
            cm = fmaf(al[n * C + m], cm, R[t][m]);
        }
    }
    __syncthreads();
    if (tid < C) {
        const int m = tid;
        float sm = 0.0f, x = 0.0f;
        for (int t = m; t < C; ++t) {
            sm = fmaf(Gam[cc + (long)t * C + m], dg[t], sm);
            x += dAl[t][m];
        }
        dal[n * C + m] = fmaf(m ? gam[n * C + m - 1] : 1.0f, sm, x);
    }
}

// dk = dku + beta gamma Z + Gamma[C-1,:] dKt; dv = beta Y (unit-major -> token-major)
__global__ __launch_bounds__(256) void ck_bwd_out_k(const float* __restrict__ dqu, const float* __restrict__ dku,
                                                    const float* __restrict__ Z, const float* __restrict__ dKt,
                                                    const float* __restrict__ Y, const float* __restrict__ be,
                                                    const float* __restrict__ gam, const float* __restrict__ gt,
                                                    int T, int H, int dh, int Tp, float* __restrict__ dq,
                                                    float* __restrict__ dk, float* __restrict__ dv, int total4) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= total4) return;
    const int hw4 = (H * dh) >> 2;
    const int col = 4 * (i % hw4);
    const int row = i / hw4;
    const int b = row / T, t = row - b * T;
    const int h = col / dh, j = col - h * dh;
    const int r = (b * H + h) * Tp + t;  // unit-major row
    const size_t o = (size_t)r * dh + j;
    const float bg = be[r] * gam[r], g = gt[r], bb = be[r];
    const float4 zq = *reinterpret_cast<const float4*>(dqu + o);
    const float4 zk = *reinterpret_cast<const float4*>(dku + o);
    const float4 zz = *reinterpret_cast<const float4*>(Z + o);
    const float4 zt = *reinterpret_cast<const float4*>(dKt + o);
    const float4 zy = *reinterpret_cast<const float4*>(Y + o);
    reinterpret_cast<float4*>(dq)[i] = zq;
    reinterpret_cast<float4*>(dk)[i] = make_float4(zk.x + bg * zz.x + g * zt.x, zk.y + bg * zz.y + g * zt.y,
                                                   zk.z + bg * zz.z + g * zt.z, zk.w + bg * zz.w + g * zt.w);
    reinterpret_cast<float4*>(dv)[i] = make_float4(bb * zy.x, bb * zy.y, bb * zy.z, bb * zy.w);
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

// Persistent state scan for dh = 128, one block per (unit, 64-column half):
//   forward  (TR = false): X_0 = 0,       X_{c+1} = G'_c   X_c + R_c, c = 0 .. NC-2
//   backward (TR = true):  X_{NC-1} = 0,  X_{c-1} = G'_c^T X_c + R_c, c = NC-1 .. 1
// X, G', R are [unit][chunk][128][128] row-major.  The block's columns are
// independent of the other half.  X^T of the block lives in LDS ([col][row],
// k-contiguous B fragments); G'_c is staged in LDS row-major, read as
// k-contiguous A fragments (forward) or as mn-contiguous A fragments
// (backward: the transpose for free), and the next chunk's G' is prefetched
// into registers during the MFMAs.  Wave w: columns 16 (w & 3) .. +15, rows
// 64 (w >> 2) .. +63 as four 16 x 16 tiles.
constexpr int SC_D = 128, SC_LD = SC_D + 4, SC_NT = 512;

template <bool TR>
__global__ __launch_bounds__(SC_NT) void ck_scan_k(const float* __restrict__ Gp, const float* __restrict__ R,
                                                   float* __restrict__ X, int NC) {
    extern __shared__ float4 sc_lds4[];
    float* As = reinterpret_cast<float*>(sc_lds4);  // [128][132]
    float* Xt = As + SC_D * SC_LD;                  // [64][132]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const long u = blockIdx.x >> 1;
    const int col0 = (blockIdx.x & 1) * 64;
    const long DD = (long)SC_D * SC_D;
    const float* Gu = Gp + u * NC * DD;
    const float* Ru = R + u * NC * DD;
    float* Xu = X + u * NC * DD;
    const int ny = w & 3, mb = (w >> 2) * 64;
    const int g4 = lane >> 4, l16 = lane & 15;
    const int ncol = 16 * ny + l16;  // column within the block's 64

    // the starting slot is zero
    const int c_first = TR ? NC - 1 : 0;
    for (int e = tid; e < 64 * SC_D; e += SC_NT) {
        const int n = e & 63, m = e >> 6;
        Xt[n * SC_LD + m] = 0.0f;
        Xu[(long)c_first * DD + (long)m * SC_D + col0 + n] = 0.0f;
    }
    if (NC < 2) return;
    // element (m, n) of this lane in tile x, register r
    auto row_of = [=](int x, int r) { return TR ? mb + 4 * (4 * g4 + r) + x : mb + 16 * x + 4 * g4 + r; };

    // G' of the next step (128 x 128 / 512 threads = 8 float4 per thread) in
    // named registers, R of the next step at this lane's 16 output elements
    float4 p0, p1, p2, p3, p4, p5, p6, p7;
    float rv[4][4];
#define SC_LOAD_G(cc)                                                                       \
    do {                                                                                    \
        const float4* src_ = reinterpret_cast<const float4*>(Gu + (long)(cc) * DD) + tid;   \
        p0 = src_[0];                                                                       \
        p1 = src_[SC_NT];                                                                   \
        p2 = src_[2 * SC_NT];                                                               \
        p3 = src_[3 * SC_NT];                                                               \
        p4 = src_[4 * SC_NT];                                                               \
        p5 = src_[5 * SC_NT];                                                               \
        p6 = src_[6 * SC_NT];                                                               \
        p7 = src_[7 * SC_NT];                                                               \
    } while (0)
#define SC_STORE_G(j, pj) \
    *reinterpret_cast<float4*>(As + ((tid + SC_NT * (j)) >> 5) * SC_LD + 4 * ((tid + SC_NT * (j)) & 31)) = (pj)
    int c = TR ? NC - 1 : 0;
    SC_LOAD_G(c);
    {
        const float* Rc = Ru + (long)c * DD;
#pragma unroll
        for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int r = 0; r < 4; ++r) rv[x][r] = Rc[(long)row_of(x, r) * SC_D + col0 + ncol];
    }
    for (int s = 0; s < NC - 1; ++s) {
        const int cn = TR ? c - 1 : c + 1;  // output slot
        __syncthreads();                     // previous step's readers of As are done
        SC_STORE_G(0, p0);
        SC_STORE_G(1, p1);
        SC_STORE_G(2, p2);
        SC_STORE_G(3, p3);
        SC_STORE_G(4, p4);
        SC_STORE_G(5, p5);
        SC_STORE_G(6, p6);
        SC_STORE_G(7, p7);
        __syncthreads();  // As and Xt ready
        f32x4 acc[4];
#pragma unroll
        for (int x = 0; x < 4; ++x) acc[x] = f32x4{rv[x][0], rv[x][1], rv[x][2], rv[x][3]};
        {
            // prefetch the next step (the last step re-reads its own chunk, unused)
            const int cl = s + 1 < NC - 1 ? cn : c;
            SC_LOAD_G(cl);
            const float* Rc = Ru + (long)cl * DD;
#pragma unroll
            for (int x = 0; x < 4; ++x)
#pragma unroll
                for (int r = 0; r < 4; ++r) rv[x][r] = Rc[(long)row_of(x, r) * SC_D + col0 + ncol];
        }
#pragma unroll
        for (int h = 0; h < SC_D / 16; ++h) {
            float fa[4][4];
            if constexpr (!TR) {
#pragma unroll
                for (int x = 0; x < 4; ++x) {
                    const float4 v = *reinterpret_cast<const float4*>(As + (mb + 16 * x + l16) * SC_LD + 16 * h + 4 * g4);
                    fa[0][x] = v.x;
                    fa[1][x] = v.y;
                    fa[2][x] = v.z;
                    fa[3][x] = v.w;
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 v = *reinterpret_cast<const float4*>(As + (16 * h + 4 * g4 + q) * SC_LD + mb + 4 * l16);
                    fa[q][0] = v.x;
                    fa[q][1] = v.y;
                    fa[q][2] = v.z;
                    fa[q][3] = v.w;
                }
            }
            const float4 b = *reinterpret_cast<const float4*>(Xt + ncol * SC_LD + 16 * h + 4 * g4);
            const float fb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int x = 0; x < 4; ++x) acc[x] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[q][x], fb[q], acc[x], 0, 0, 0);
        }
        __syncthreads();  // every wave has read Xt
        float* Xn = Xu + (long)cn * DD;
#pragma unroll
        for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = row_of(x, r);
                Xt[ncol * SC_LD + m] = acc[x][r];
                Xn[(long)m * SC_D + col0 + ncol] = acc[x][r];
            }
        c = cn;
    }
#undef SC_LOAD_G
#undef SC_STORE_G
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
    const ChunkDims d = chunk_dims(B, T, H, dh, C);
    if (d.U * d.Tp * dh >= (1L << 31) || d.N * d.DD >= (1L << 31) || (long)B * T * H * dh >= (1L << 31))
        return fail(ASCA_ERR_UNSUPPORTED, "chunked: tensors beyond 2^31 elements");
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

// As CK_LAUNCH with dynamic LDS (at most 64 KB: no attribute needed).
#define CK_LAUNCH_LDS(name, kern, grid, block, lds, ...)             \
    do {                                                             \
        int rc_ = pre_launch(name);                                  \
        if (rc_) return rc_;                                         \
        hipLaunchKernelGGL(kern, grid, block, lds, st, __VA_ARGS__); \
        rc_ = post_launch(name);                                     \
        if (rc_) return rc_;                                         \
    } while (0)

// ---------------------------------------------------------------- fused prep
// One block per chunk for C = 64, dh = 128: everything of a chunk that does
// not depend on the state, with the chunk's operands in LDS and every product
// on the matrix cores through wave_mm.  It writes the workspace arrays that
// the factorised scan (ck_scan2_k), the output kernel and the fused backward
// read; G' and H of the decomposed path are not formed (the scan works from W
// and Kt directly).
constexpr int FP_C = 64, FP_D = 128, FP_LK = FP_D + 4, FP_LC = FP_C + 4, FP_NT = 512;
constexpr int FP_LDS_F = 3 * FP_C * FP_LK + 2 * FP_C * FP_LC + 5 * FP_C + 8 * FP_C;

// Four k-consecutive elements of an LDS operand at (mn, k .. k+3): element
// (mn, k) at P[mn*ld + k] if KC (one 8- or 16-byte read) else P[k*ld + mn];
// BF: the operand is stored as bf16 (exact for bf16 inputs), else f32.
template <bool KC, bool BF>
ASCA_DEV f32x4 lds_frag(const void* P, int ld, int mn, int k) {
    f32x4 r;
    if constexpr (BF) {
        const uint16_t* p = reinterpret_cast<const uint16_t*>(P);
        if constexpr (KC) {
            const uint2 x = *reinterpret_cast<const uint2*>(p + mn * ld + k);
            r = f32x4{__uint_as_float(x.x << 16), __uint_as_float(x.x & 0xffff0000u), __uint_as_float(x.y << 16),
                      __uint_as_float(x.y & 0xffff0000u)};
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) r[s] = __uint_as_float((uint32_t)p[(k + s) * ld + mn] << 16);
        }
    } else {
        const float* p = reinterpret_cast<const float*>(P);
        if constexpr (KC) {
            r = *reinterpret_cast<const f32x4*>(p + mn * ld + k);
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) r[s] = p[(k + s) * ld + mn];
        }
    }
    return r;
}

// acc[TM][TN] (16 x 16 tiles at rows m0 + 16x, columns n0 + 16y) += op(A) op(B)
// over k in [k_lo, k_hi) (a multiple of 16), operands in LDS.  A element
// (m, k) is A[m*lda + k] if AK (contiguous in k) else A[k*lda + m]; B element
// (k, n) is B[n*ldb + k] if BK else B[k*ldb + n]; AB / BB: bf16 storage;
// optional per-k scales sa[k], sb[k].  Within each 16-k block lane l feeds k =
// 4(l/16) + s at step s of v_mfma_f32_16x16x4_f32 (any order of k gives the
// same sum), so an operand contiguous in k is one 8- or 16-byte read.
template <int TM, int TN, bool AK, bool AB, bool BK, bool BB, bool SA = false, bool SB = false>
ASCA_DEV void wave_mm(f32x4 (&acc)[TM][TN], int k_lo, int k_hi, const void* A, int lda, const float* sa,
                      const void* B, int ldb, const float* sb, int m0, int n0, int lane) {
    const int li = lane & 15, kq = lane >> 4;
    // fragments of the 16-k block at kb (clamped into the range: a block read
    // past the end is never multiplied)
    auto frag = [&](int kb, f32x4 (&a)[TM], f32x4 (&b)[TN]) {
        const int k = min(kb, k_hi - 16) + 4 * kq;
#pragma unroll
        for (int x = 0; x < TM; ++x) {
            a[x] = lds_frag<AK, AB>(A, lda, m0 + 16 * x + li, k);
            if (SA) a[x] *= *reinterpret_cast<const f32x4*>(sa + k);
        }
#pragma unroll
        for (int y = 0; y < TN; ++y) {
            b[y] = lds_frag<BK, BB>(B, ldb, n0 + 16 * y + li, k);
            if (SB) b[y] *= *reinterpret_cast<const f32x4*>(sb + k);
        }
    };
    auto mm = [&](const f32x4 (&a)[TM], const f32x4 (&b)[TN]) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int x = 0; x < TM; ++x)
#pragma unroll
                for (int y = 0; y < TN; ++y)
                    acc[x][y] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[x][s], b[y][s], acc[x][y], 0, 0, 0);
    };
    if (k_hi <= k_lo) return;
    // Software-pipelined: the fragments of the next 16-k block are read before
    // the products of the current one, which hide the reads' latency (the
    // scheduling barriers keep the compiler from sinking the reads to their use).
    f32x4 a0[TM], b0[TN], a1[TM], b1[TN];
    frag(k_lo, a0, b0);
    int kb = k_lo;
    for (; kb + 32 <= k_hi; kb += 32) {
        frag(kb + 16, a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        mm(a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        frag(kb + 32, a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        mm(a1, b1);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (kb < k_hi) mm(a0, b0);   // an odd last block
}

template <int TM, int TN>
ASCA_DEV void acc_zero(f32x4 (&acc)[TM][TN]) {
#pragma unroll
    for (int x = 0; x < TM; ++x)
#pragma unroll
        for (int y = 0; y < TN; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// Streaming stores for workspace arrays read back only by later kernels.
ASCA_DEV void st_nt(float* p, float v) { __builtin_nontemporal_store(v, p); }
ASCA_DEV void st_nt4(float* p, float4 v) {
    __builtin_nontemporal_store(f32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4*>(p));
}

// 4 bf16 of chunk row t at column f, 0 for rows past the sequence (t >=
// valid, valid >= 1).  The load itself is unconditional (row clamped): a load
// under a branch is waited for inside the branch, which serialises the loads.
ASCA_DEV uint2 ld_row4(const uint16_t* __restrict__ src, long rowbase, long rowstride, int t, int valid, int f) {
    const uint2 x = *reinterpret_cast<const uint2*>(src + rowbase + (long)min(t, valid - 1) * rowstride + f);
    return t < valid ? x : make_uint2(0u, 0u);
}

ASCA_DEV float4 bf4_f32(uint2 r) {
    return make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u), __uint_as_float(r.y << 16),
                       __uint_as_float(r.y & 0xffff0000u));
}

// A chunk's rows held as bf16 in registers (the zero rows past T included), by
// all FP_NT threads, so that a tensor needed in LDS twice, or later than it is
// loaded, is read from HBM once and early.
struct FpRows {
    uint2 r[FP_C * FP_D / 4 / FP_NT];
};

ASCA_DEV void fp_rows_ld(FpRows& x, const uint16_t* __restrict__ src, long rowbase, long rowstride, int valid_rows,
                         int tid) {
#pragma unroll
    for (int i = 0; i < (int)(sizeof(x.r) / sizeof(x.r[0])); ++i) {
        const int e = tid + i * FP_NT;
        x.r[i] = ld_row4(src, rowbase, rowstride, e >> 5, valid_rows, 4 * (e & 31));
    }
}

ASCA_DEV void fp_rows_st(const FpRows& x, float* lds, int tid) {
#pragma unroll
    for (int i = 0; i < (int)(sizeof(x.r) / sizeof(x.r[0])); ++i) {
        const int e = tid + i * FP_NT;
        *reinterpret_cast<float4*>(lds + (e >> 5) * FP_LK + 4 * (e & 31)) = bf4_f32(x.r[i]);
    }
}

// Off-diagonal 16 x 16 block (i, j), i > j, of T = (I + L)^-1 from the blocks
// already known: T_ij = -T_ii (L[i, j..i) T[j..i, j]), one wave.  Ls holds L,
// Ts holds T (both stride FP_LC).  The product's accumulator feeds the second
// product directly as its B operand (lane l, register s = row 4(l/16) + s).
ASCA_DEV void fp_tri_block(const float* Ls, float* Ts, int i, int j, int lane) {
    const int li = lane & 15, kq = lane >> 4;
    f32x4 x[1][1];
    acc_zero(x);
    wave_mm<1, 1, true, false, false, false, false, false>(x, 16 * j, 16 * i, Ls, FP_LC, nullptr, Ts, FP_LC, nullptr, 16 * i, 16 * j,
                                             lane);
    const f32x4 d = *reinterpret_cast<const f32x4*>(Ts + (16 * i + li) * FP_LC + 16 * i + 4 * kq);
    f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) y = __builtin_amdgcn_mfma_f32_16x16x4f32(d[s], x[0][0][s], y, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) Ts[(16 * i + 4 * kq + r) * FP_LC + 16 * j + li] = -y[r];
}

__global__ __launch_bounds__(FP_NT) void ck_fwd_prep_k(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                       const uint16_t* __restrict__ v, const float* __restrict__ alpha,
                                                       const float* __restrict__ beta, int T, int H, int NC, ChunkWs w) {
    extern __shared__ float4 fp_lds4[];
    float* const Ks = reinterpret_cast<float*>(fp_lds4);  // K           [64][132]
    float* const X = Ks + FP_C * FP_LK;                    // Q, then V, then Q
    float* const Y = X + FP_C * FP_LK;                     // Gamma, then T [64][68]; then W [64][132]
    float* const Ls = Y + FP_C * FP_LK;                    // L, then T  [64][68]
    float* const Ms = Ls + FP_C * FP_LC;                   // M          [64][68]
    float* const a_s = Ms + FP_C * FP_LC;
    float* const b_s = a_s + FP_C;
    float* const g_s = b_s + FP_C;
    float* const gt_s = g_s + FP_C;
    float* const bg_s = gt_s + FP_C;
    float* const seg_s = bg_s + FP_C;  // [8][64] per-segment products of Gamma's columns
    float* const Gs = Y;
    float* const Ts = Y;

    const long n = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int li = lane & 15, l4 = lane >> 4;
    const long u = n / NC;
    const int c = (int)(n - u * NC);
    const int b = (int)(u / H), h = (int)(u - (long)b * H);
    const int t0 = c * FP_C;
    const int valid = min(FP_C, T - t0);
    const long rowbase = ((long)b * T + t0) * H * FP_D + (long)h * FP_D;
    const long rowstride = (long)H * FP_D;
    const long cd = n * FP_C * FP_D, cc = n * FP_C * FP_C, dd = n * FP_D * FP_D;

    // gates (padding steps are identities), K and Q into LDS; Q and V stay in
    // registers for later (every row load of the kernel is in flight here)
    FpRows kr, qr, vr;
    fp_rows_ld(kr, k, rowbase, rowstride, valid, tid);
    fp_rows_ld(qr, q, rowbase, rowstride, valid, tid);
    fp_rows_ld(vr, v, rowbase, rowstride, valid, tid);
    fp_rows_st(kr, Ks, tid);
    fp_rows_st(qr, X, tid);
    if (tid < FP_C) {
        const bool in = tid < valid;
        const long gi = ((long)b * T + t0 + min(tid, valid - 1)) * H + h;
        const float av = alpha[gi], bv = beta[gi];
        a_s[tid] = in ? av : 1.0f;
        b_s[tid] = in ? bv : 0.0f;
        w.al[n * FP_C + tid] = in ? av : 1.0f;
        w.be[n * FP_C + tid] = in ? bv : 0.0f;
    }
    __syncthreads();
    // gamma: inclusive product scan over the first wave.  Gamma[t][i] =
    // prod_{i < s <= t} alpha_s (t >= i), never by division (gamma can
    // underflow): thread (column i, segment sg) forms the running products of
    // rows 8 sg .. 8 sg + 7, then scales them by the product of the column's
    // earlier segments.
    if (tid < FP_C) {
        float g = a_s[tid];
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_up(g, o);
            if (tid >= o) g *= y;
        }
        g_s[tid] = g;
    }
    {
        const int i = tid & 63, sg = tid >> 6;
        float x = 1.0f;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int t = 8 * sg + r;
            if (t > i) x *= a_s[t];
            Gs[t * FP_LC + i] = t >= i ? x : 0.0f;
        }
        seg_s[sg * 64 + i] = x;
    }
    __syncthreads();
    {
        const int i = tid & 63, sg = tid >> 6;
        float pre = 1.0f;
        for (int s2 = 0; s2 < sg; ++s2) pre *= seg_s[s2 * 64 + i];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int t = 8 * sg + r;
            const float val = Gs[t * FP_LC + i] * pre;
            Gs[t * FP_LC + i] = val;
            w.Gam[cc + t * FP_C + i] = val;
        }
        if (sg == 7) gt_s[i] = pre * seg_s[7 * 64 + i];
    }
    __syncthreads();
    if (tid < FP_C) {
        w.gam[n * FP_C + tid] = g_s[tid];
        w.gt[n * FP_C + tid] = gt_s[tid];
        bg_s[tid] = b_s[tid] * g_s[tid];
    }
    if (tid == 0) w.gC[n] = g_s[FP_C - 1];
    // A = K K^T -> L = strict_tril(beta_j Gamma A);  B = Q K^T -> M = tril(Gamma B)
    {
        const int m0 = 16 * (wv >> 1), n0 = 32 * (wv & 1);
        f32x4 aa[1][2], ab[1][2];
        acc_zero(aa);
        acc_zero(ab);
        wave_mm<1, 2, true, false, true, false, false, false>(aa, 0, FP_D, Ks, FP_LK, nullptr, Ks, FP_LK, nullptr, m0, n0, lane);
        wave_mm<1, 2, true, false, true, false, false, false>(ab, 0, FP_D, X, FP_LK, nullptr, Ks, FP_LK, nullptr, m0, n0, lane);
#pragma unroll
        for (int y = 0; y < 2; ++y)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int j = m0 + 4 * l4 + r, i = n0 + 16 * y + li;
                const float g = Gs[j * FP_LC + i];
                const float va = aa[0][y][r], vb = ab[0][y][r];
                w.Am[cc + j * FP_C + i] = va;
                w.Bm[cc + j * FP_C + i] = vb;
                Ls[j * FP_LC + i] = i < j ? b_s[j] * (g * va) : 0.0f;
                const float mv = i <= j ? g * vb : 0.0f;
                Ms[j * FP_LC + i] = mv;
                w.Mm[cc + j * FP_C + i] = mv;
            }
    }
    __syncthreads();
    // T = (I + L)^-1 into Ts.  First wave: the four 16 x 16 diagonal blocks,
    // lane = (block, column), the column in registers, right-looking forward
    // substitution.  The other waves zero the blocks above the diagonal; then
    // V (in registers since the start) goes where Q was.  (Kt = Gamma[C-1, :] K
    // is not stored: the fused backward forms it from K and Gamma[C-1, :].)
    if (wv == 0) {
        const int o = 16 * l4, m = li;
        float d[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) d[r] = r == m ? 1.0f : 0.0f;
#pragma unroll
        for (int jj = 0; jj < 15; ++jj)
#pragma unroll
            for (int r = jj + 1; r < 16; ++r) d[r] -= Ls[(o + r) * FP_LC + o + jj] * d[jj];
#pragma unroll
        for (int r = 0; r < 16; ++r) Ts[(o + r) * FP_LC + o + m] = d[r];
    } else {
        const int t2 = tid - 64;
        for (int e = t2; e < 6 * 256; e += FP_NT - 64) {  // blocks (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
            const int blk = e >> 8, bi = blk < 3 ? 0 : (blk < 5 ? 1 : 2);
            const int bj = blk < 3 ? blk + 1 : (blk < 5 ? blk - 1 : 3);
            Ts[(16 * bi + ((e >> 4) & 15)) * FP_LC + 16 * bj + (e & 15)] = 0.0f;
        }
    }
    fp_rows_st(vr, X, tid);   // Q's reads are done (the barrier before this phase)
    __syncthreads();
    // the blocks below the diagonal, one block diagonal at a time
    if (wv < 3) fp_tri_block(Ls, Ts, wv + 1, wv, lane);
    __syncthreads();
    if (wv < 2) fp_tri_block(Ls, Ts, wv + 2, wv, lane);
    __syncthreads();
    if (wv == 0) fp_tri_block(Ls, Ts, 3, 0, lane);
    __syncthreads();
    for (int e = tid; e < FP_C * FP_C; e += FP_NT) {
        const float t = Ts[(e >> 6) * FP_LC + (e & 63)];
        Ls[(e >> 6) * FP_LC + (e & 63)] = t;
        w.Tm[cc + e] = t;
    }
    __syncthreads();
    // Uv = T diag(beta) V -> the workspace
    {
        const int m0 = 32 * (wv >> 2), n0 = 32 * (wv & 3);
        f32x4 acc[2][2];
        acc_zero(acc);
        wave_mm<2, 2, true, false, false, false, false, true>(acc, 0, FP_C, Ls, FP_LC, nullptr, X, FP_LK, b_s, m0, n0, lane);
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
            for (int y = 0; y < 2; ++y)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = m0 + 16 * x + 4 * l4 + r, f = n0 + 16 * y + li;
                    st_nt(w.Uv + cd + t * FP_D + f, acc[x][y][r]);
                }
    }
    __syncthreads();  // every read of V is done before Q comes back into X
    // W = T diag(beta gamma) K -> Y; Q back into X
    {
        const int m0 = 32 * (wv >> 2), n0 = 32 * (wv & 3);
        f32x4 acc[2][2];
        acc_zero(acc);
        wave_mm<2, 2, true, false, false, false, false, true>(acc, 0, FP_C, Ls, FP_LC, nullptr, Ks, FP_LK, bg_s, m0, n0, lane);
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
            for (int y = 0; y < 2; ++y)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = m0 + 16 * x + 4 * l4 + r, f = n0 + 16 * y + li;
                    Y[t * FP_LK + f] = acc[x][y][r];
                    st_nt(w.W + cd + t * FP_D + f, acc[x][y][r]);
                }
        fp_rows_st(qr, X, tid);
    }
    __syncthreads();
    // Qp = diag(gamma) Q - M W
    {
        const int m0 = 32 * (wv >> 2), n0 = 32 * (wv & 3);
        f32x4 acc[2][2];
        acc_zero(acc);
        wave_mm<2, 2, true, false, false, false, false, false>(acc, 0, FP_C, Ms, FP_LC, nullptr, Y, FP_LK, nullptr, m0, n0, lane);
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
            for (int y = 0; y < 2; ++y)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = m0 + 16 * x + 4 * l4 + r, f = n0 + 16 * y + li;
                    st_nt(w.Qp + cd + t * FP_D + f, g_s[t] * X[t * FP_LK + f] - acc[x][y][r]);
                }
    }
}

// ---------------------------------------------------------------- fused backward
// One block per chunk for C = 64, dh = 128, after the reverse state scan: all
// per-chunk gradients of q, k, v, alpha, beta, written token-major.  It uses
//   Z = T^T dW = -Y S^T          (dW = -dU S^T, Y = T^T dU)
//   dL = -strict_tril(Y Uv^T + Z W^T) = -strict_tril(Y U^T)   (U = Uv - W S)
//   dO_t . (Q S)_t = Q_t . (dO S^T)_t
// so neither dW nor Q S is formed.  The 128 x 128 states S and dS' pass through
// LDS in 64-row halves; K, Q, dO sit in LDS as bf16 (exact: they are bf16
// inputs).  Wave w owns rows 16 (w >> 1) .. +15 of every C x dh result and the
// columns 32 (w & 1) + {0, 16} of each 64-column half, so the halves of the
// state products never leave a wave idle.
constexpr int FB_LB = FP_D + 8;              // bf16 row stride of the [64][128] bf16 operands
constexpr int FB_BIG = FP_C * FP_LK;         // f32 [64][132]
constexpr int FB_SMALL = FP_C * FP_LC;       // f32 [64][68], or bf16 [64][136]
constexpr int FB_LDS_F = 3 * FB_BIG + 3 * FB_SMALL + 1536;

ASCA_DEV float bf_at(const uint16_t* p, int i) { return __uint_as_float((uint32_t)p[i] << 16); }

ASCA_DEV float sum16(float x) {
    x += __shfl_xor(x, 1);
    x += __shfl_xor(x, 2);
    x += __shfl_xor(x, 4);
    x += __shfl_xor(x, 8);
    return x;
}

// Row partials p[r] of a wave's 16-row strip (row m0 + 4 (lane / 16) + r)
// summed over the 16 lanes of a row -> dst[row].
ASCA_DEV void rows_out(const float (&p)[4], float* dst, int m0, int lane) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float x = sum16(p[r]);
        if ((lane & 15) == 0) dst[m0 + 4 * (lane >> 4) + r] = x;
    }
}

// 64 rows x 128 f32 from global (row stride 128) into LDS (row stride FP_LK).
ASCA_DEV void fb_rows_f32(const float* __restrict__ src, float* dst, int tid) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = tid + i * FP_NT, r = e >> 5, f = 4 * (e & 31);
        *reinterpret_cast<float4*>(dst + r * FP_LK + f) = *reinterpret_cast<const float4*>(src + r * FP_D + f);
    }
}

// 64 x 64 f32 (row stride ld_src) into LDS (row stride FP_LC).
ASCA_DEV void fb_sq_f32(const float* __restrict__ src, int ld_src, float* dst, int tid) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int e = tid + i * FP_NT, r = e >> 4, f = 4 * (e & 15);
        *reinterpret_cast<float4*>(dst + r * FP_LC + f) = *reinterpret_cast<const float4*>(src + r * ld_src + f);
    }
}

__global__ __launch_bounds__(FP_NT) void ck_bwd_fused_k(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                        const uint16_t* __restrict__ v,
                                                        const uint16_t* __restrict__ d_o, int T, int H, int NC,
                                                        ChunkWs w, float* __restrict__ dq, float* __restrict__ dk,
                                                        float* __restrict__ dv, float* __restrict__ dalpha,
                                                        float* __restrict__ dbeta) {
    extern __shared__ float4 fb_lds4[];
    float* const RA = reinterpret_cast<float*>(fb_lds4);  // S / dS' halves; T; GdM | dA
    float* const RB = RA + FB_BIG;                         // dS' half; U
    float* const RC = RB + FB_BIG;                         // dU, then Y
    float* const RE = RC + FB_BIG;                         // W half; M; R; Q (bf16)
    uint16_t* const Kb = reinterpret_cast<uint16_t*>(RE + FB_SMALL);
    uint16_t* const Ob = reinterpret_cast<uint16_t*>(RE + 2 * FB_SMALL);
    uint16_t* const Qb = reinterpret_cast<uint16_t*>(RE);
    float* const a_s = RE + 3 * FB_SMALL;
    float* const b_s = a_s + 64;
    float* const g_s = b_s + 64;
    float* const gt_s = g_s + 64;
    float* const pz = gt_s + 64;  // [2][64] row partials: Z.K
    float* const pk = pz + 128;   // K.dKt
    float* const pq = pk + 128;   // Q.(dO S^T)
    float* const pyv = pq + 128;  // Y.V
    float* const ppb = pyv + 128; // sum_i dL Gamma A
    float* const pr = ppb + 128;  // [8][64] partials of the R term of d log alpha
    float* const dlr = pr + 512;
    float* const fr = dlr + 64;   // [8]

    const long n = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int li = lane & 15, l4 = lane >> 4;
    const long u = n / NC;
    const int c = (int)(n - u * NC);
    const int b = (int)(u / H), h = (int)(u - (long)b * H);
    const int t0 = c * FP_C;
    const int valid = min(FP_C, T - t0);
    const long rowbase = ((long)b * T + t0) * H * FP_D + (long)h * FP_D;
    const long rowstride = (long)H * FP_D;
    const long cd = n * FP_C * FP_D, cc = n * FP_C * FP_C, dd = n * FP_D * FP_D;
    const int rm0 = 16 * (wv >> 1), cn0 = 32 * (wv & 1);

    if (tid < FP_C) {
        a_s[tid] = w.al[n * FP_C + tid];
        b_s[tid] = w.be[n * FP_C + tid];
        g_s[tid] = w.gam[n * FP_C + tid];
        gt_s[tid] = w.gt[n * FP_C + tid];
    }
    {   // K and dO rows (bf16, exact), zero past T; every load issued first
        uint2 xk[4], xo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = tid + i * FP_NT, t = e >> 5, f = 4 * (e & 31);
            xk[i] = ld_row4(k, rowbase, rowstride, t, valid, f);
            xo[i] = ld_row4(d_o, rowbase, rowstride, t, valid, f);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = tid + i * FP_NT, t = e >> 5, f = 4 * (e & 31);
            *reinterpret_cast<uint2*>(Kb + t * FB_LB + f) = xk[i];
            *reinterpret_cast<uint2*>(Ob + t * FB_LB + f) = xo[i];
        }
    }

    // ---- dU = diag(gt) K dS' + M^T dO over the two row halves of dS'; U = Uv - W S
    // was stored by the forward scan
    f32x4 D0[1][2], D1[1][2];
    acc_zero(D0);
    acc_zero(D1);
    float fro = 0.0f;
    fb_sq_f32(w.Mm + cc, FP_C, RE, tid);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        fb_rows_f32(w.dSp + dd + 64 * hh * FP_D, RB, tid);
        __syncthreads();
        wave_mm<1, 2, true, true, false, false>(D0, 0, 64, Kb + 64 * hh, FB_LB, nullptr, RB, FP_LK, nullptr, rm0, cn0,
                                                lane);
        wave_mm<1, 2, true, true, false, false>(D1, 0, 64, Kb + 64 * hh, FB_LB, nullptr, RB, FP_LK, nullptr, rm0,
                                                64 + cn0, lane);
        __syncthreads();
    }
    fb_sq_f32(w.Tm + cc, FP_C, RA, tid);
    fb_rows_f32(w.Uu + cd, RB, tid);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float g = gt_s[rm0 + 4 * l4 + r];
#pragma unroll
        for (int y = 0; y < 2; ++y) {
            D0[0][y][r] *= g;
            D1[0][y][r] *= g;
        }
    }
    wave_mm<1, 2, false, false, false, true>(D0, 0, 64, RE, FP_LC, nullptr, Ob, FB_LB, nullptr, rm0, cn0, lane);
    wave_mm<1, 2, false, false, false, true>(D1, 0, 64, RE, FP_LC, nullptr, Ob, FB_LB, nullptr, rm0, 64 + cn0, lane);
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
        for (int y = 0; y < 2; ++y)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = rm0 + 4 * l4 + r, f = 64 * g2 + cn0 + 16 * y + li;
                RC[t * FP_LK + f] = g2 ? D1[0][y][r] : D0[0][y][r];
            }
    __syncthreads();

    // ---- Y = T^T dU; dv = beta Y
    {
        // V at this lane's Y positions; a whole chunk (every chunk but a ragged
        // last one) takes the branch without a per-row condition, so its 16
        // loads are all in flight together
        float pV[2][2][4];
        if (valid == FP_C) {
#pragma unroll
            for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
                for (int y = 0; y < 2; ++y)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        pV[g2][y][r] = __uint_as_float(
                            (uint32_t)v[rowbase + (long)(rm0 + 4 * l4 + r) * rowstride + 64 * g2 + cn0 + 16 * y + li]
                            << 16);
        } else {
#pragma unroll
            for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
                for (int y = 0; y < 2; ++y)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int t = rm0 + 4 * l4 + r;
                        pV[g2][y][r] = t < valid ? __uint_as_float((uint32_t)v[rowbase + (long)t * rowstride + 64 * g2 +
                                                                               cn0 + 16 * y + li]
                                                                   << 16)
                                                 : 0.0f;
                    }
        }
        f32x4 Y0[1][2], Y1[1][2];
        acc_zero(Y0);
        acc_zero(Y1);
        wave_mm<1, 2, false, false, false, false>(Y0, 0, 64, RA, FP_LC, nullptr, RC, FP_LK, nullptr, rm0, cn0, lane);
        wave_mm<1, 2, false, false, false, false>(Y1, 0, 64, RA, FP_LC, nullptr, RC, FP_LK, nullptr, rm0, 64 + cn0,
                                                  lane);
        float yv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
            for (int y = 0; y < 2; ++y)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = rm0 + 4 * l4 + r, f = 64 * g2 + cn0 + 16 * y + li;
                    const float yy = g2 ? Y1[0][y][r] : Y0[0][y][r];
                    if (t < valid) dv[rowbase + (long)t * rowstride + f] = b_s[t] * yy;
                    yv[r] += yy * pV[g2][y][r];
                }
        rows_out(yv, pyv + 64 * (wv & 1), rm0, lane);
        __syncthreads();  // every read of dU and T is done
#pragma unroll
        for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
            for (int y = 0; y < 2; ++y)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = rm0 + 4 * l4 + r, f = 64 * g2 + cn0 + 16 * y + li;
                    RC[t * FP_LK + f] = g2 ? Y1[0][y][r] : Y0[0][y][r];
                }
    }
    __syncthreads();

    // ---- dM = tril(dO U^T), dL = -strict_tril(Y U^T) -> GdM, dA (RA), R (RE), row sums of dL Gamma A
    {
        float pGa[2][4], pAm[2][4], pBm[2][4];
#pragma unroll
        for (int y = 0; y < 2; ++y)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const long o = cc + (rm0 + 4 * l4 + r) * FP_C + cn0 + 16 * y + li;
                pGa[y][r] = w.Gam[o];
                pAm[y][r] = w.Am[o];
                pBm[y][r] = w.Bm[o];
            }
        f32x4 Mx[1][2], Lx[1][2];
        acc_zero(Mx);
        acc_zero(Lx);
        wave_mm<1, 2, true, true, true, false>(Mx, 0, FP_D, Ob, FB_LB, nullptr, RB, FP_LK, nullptr, rm0, cn0, lane);
        wave_mm<1, 2, true, false, true, false>(Lx, 0, FP_D, RC, FP_LK, nullptr, RB, FP_LK, nullptr, rm0, cn0, lane);
        float pb[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int y = 0; y < 2; ++y)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int j = rm0 + 4 * l4 + r, i = cn0 + 16 * y + li;
                const float g = pGa[y][r], am = pAm[y][r], bj = b_s[j];
                const float dm = i <= j ? Mx[0][y][r] : 0.0f;
                const float dl = i < j ? -Lx[0][y][r] : 0.0f;
                RA[j * FP_LK + i] = g * dm;
                RA[j * FP_LK + 64 + i] = dl * bj * g;
                const float dG = dm * pBm[y][r] + dl * bj * am;
                RE[j * FP_LC + i] = i < j ? dG : 0.0f;   // dGamma, strictly lower
                pb[r] += dl * g * am;
            }
        rows_out(pb, ppb + 64 * (wv & 1), rm0, lane);
    }
    // Q (exact in bf16) staged in registers while R is reduced
    uint2 qst[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = tid + i * FP_NT, r = e >> 5, f = 4 * (e & 31);
        qst[i] = ld_row4(q, rowbase, rowstride, r, valid, f);
    }
    __syncthreads();
    // dGamma term of dalpha_m (no division, exact at alpha_m = 0):
    //   sum_{t >= m} Gamma[t][m] c_t(m),  c_t(m) = sum_{i < m} dGamma[t][i] Gamma[m-1][i],
    // c_t(m+1) = alpha_m c_t(m) + dGamma[t][m] as an affine scan over the lanes;
    // wave w takes rows 8w .. 8w+7
    {
        float gr[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) gr[r] = w.Gam[cc + (long)(8 * wv + r) * FP_C + lane];
        // the scan's multipliers (products of alpha over the lanes' windows) are the same for every row
        float am[6];
        {
            float a = a_s[lane];
#pragma unroll
            for (int lv = 0, o = 1; o < 64; o <<= 1, ++lv) {
                am[lv] = a;
                const float ap = __shfl_up(a, o);
                if (lane >= o) a *= ap;
            }
        }
        float acc = 0.0f;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int t = 8 * wv + r;
            float x = RE[t * FP_LC + lane];
#pragma unroll
            for (int lv = 0, o = 1; o < 64; o <<= 1, ++lv) {
                const float xp = __shfl_up(x, o);
                if (lane >= o) x = fmaf(am[lv], xp, x);
            }
            float cm = __shfl_up(x, 1);   // x = c_t(lane + 1)
            if (lane == 0) cm = 0.0f;
            if (t >= lane) acc = fmaf(gr[r], cm, acc);
        }
        pr[wv * 64 + lane] = acc;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = tid + i * FP_NT, r = e >> 5, f = 4 * (e & 31);
        *reinterpret_cast<uint2*>(Qb + r * FB_LB + f) = qst[i];
    }
    if (tid < 64) {
        float sacc = 0.0f;
#pragma unroll
        for (int k2 = 0; k2 < 8; ++k2) sacc += pr[k2 * 64 + tid];
        dlr[tid] = sacc;
    }
    __syncthreads();

    // ---- dq = GdM K (+ gamma dO S^T below); dk = GdM^T Q + (dA + dA^T) K (+ beta gamma Z + gt dKt below)
    f32x4 Q0[1][2], Q1[1][2], K0[1][2], K1[1][2];
    acc_zero(Q0);
    acc_zero(Q1);
    acc_zero(K0);
    acc_zero(K1);
    wave_mm<1, 2, true, false, false, true>(Q0, 0, 64, RA, FP_LK, nullptr, Kb, FB_LB, nullptr, rm0, cn0, lane);
    wave_mm<1, 2, true, false, false, true>(Q1, 0, 64, RA, FP_LK, nullptr, Kb, FB_LB, nullptr, rm0, 64 + cn0, lane);
    wave_mm<1, 2, false, false, false, true>(K0, 0, 64, RA, FP_LK, nullptr, Qb, FB_LB, nullptr, rm0, cn0, lane);
    wave_mm<1, 2, false, false, false, true>(K1, 0, 64, RA, FP_LK, nullptr, Qb, FB_LB, nullptr, rm0, 64 + cn0, lane);
    wave_mm<1, 2, true, false, false, true>(K0, 0, 64, RA + 64, FP_LK, nullptr, Kb, FB_LB, nullptr, rm0, cn0, lane);
    wave_mm<1, 2, true, false, false, true>(K1, 0, 64, RA + 64, FP_LK, nullptr, Kb, FB_LB, nullptr, rm0, 64 + cn0,
                                            lane);
    wave_mm<1, 2, false, false, false, true>(K0, 0, 64, RA + 64, FP_LK, nullptr, Kb, FB_LB, nullptr, rm0, cn0, lane);
    wave_mm<1, 2, false, false, false, true>(K1, 0, 64, RA + 64, FP_LK, nullptr, Kb, FB_LB, nullptr, rm0, 64 + cn0,
                                             lane);
    __syncthreads();

    // ---- per row half of S and dS': Z = -Y S^T, P = dO S^T, dKt = U dS'^T (columns of that half)
    float zk[4] = {0.f, 0.f, 0.f, 0.f}, kk[4] = {0.f, 0.f, 0.f, 0.f}, qd[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        fb_rows_f32(w.S + dd + 64 * hh * FP_D, RA, tid);
        __syncthreads();
        f32x4 Zx[1][2], Px[1][2], Tx[1][2];
        acc_zero(Zx);
        acc_zero(Px);
        acc_zero(Tx);
        wave_mm<1, 2, true, false, true, false>(Zx, 0, FP_D, RC, FP_LK, nullptr, RA, FP_LK, nullptr, rm0, cn0, lane);
        wave_mm<1, 2, true, true, true, false>(Px, 0, FP_D, Ob, FB_LB, nullptr, RA, FP_LK, nullptr, rm0, cn0, lane);
        __syncthreads();
        // dS' half over the S half, <S, dS'> on the way (each thread reads
        // the S elements it then overwrites)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = tid + i * FP_NT, r = e >> 5, f = 4 * (e & 31);
            const float4 gv = *reinterpret_cast<const float4*>(w.dSp + dd + (long)(64 * hh + r) * FP_D + f);
            const float4 sv = *reinterpret_cast<const float4*>(RA + r * FP_LK + f);
            fro += (sv.x * gv.x + sv.y * gv.y) + (sv.z * gv.z + sv.w * gv.w);
            *reinterpret_cast<float4*>(RA + r * FP_LK + f) = gv;
        }
        __syncthreads();
        wave_mm<1, 2, true, false, true, false>(Tx, 0, FP_D, RB, FP_LK, nullptr, RA, FP_LK, nullptr, rm0, cn0, lane);
#pragma unroll
        for (int y = 0; y < 2; ++y)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = rm0 + 4 * l4 + r, a = 64 * hh + cn0 + 16 * y + li;
                const float z = -Zx[0][y][r], pp = Px[0][y][r], dkt = Tx[0][y][r];
                const float kv = bf_at(Kb, t * FB_LB + a), qv = bf_at(Qb, t * FB_LB + a);
                zk[r] += z * kv;
                kk[r] += kv * dkt;
                qd[r] += qv * pp;
                const float dqv = g_s[t] * pp, dkv = (b_s[t] * g_s[t]) * z + gt_s[t] * dkt;
                if (hh) {
                    Q1[0][y][r] += dqv;
                    K1[0][y][r] += dkv;
                } else {
                    Q0[0][y][r] += dqv;
                    K0[0][y][r] += dkv;
                }
            }
        __syncthreads();
    }

    // ---- outputs
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
        for (int y = 0; y < 2; ++y)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = rm0 + 4 * l4 + r, a = 64 * g2 + cn0 + 16 * y + li;
                if (t < valid) {
                    const long o = rowbase + (long)t * rowstride + a;
                    dq[o] = g2 ? Q1[0][y][r] : Q0[0][y][r];
                    dk[o] = g2 ? K1[0][y][r] : K0[0][y][r];
                }
            }
    rows_out(zk, pz + 64 * (wv & 1), rm0, lane);
    rows_out(kk, pk + 64 * (wv & 1), rm0, lane);
    rows_out(qd, pq + 64 * (wv & 1), rm0, lane);
    fro = wave_sum(fro);
    if (lane == 0) fr[wv] = fro;
    __syncthreads();
    if (wv == 0) {
        const int t = lane;
        const float zkt = pz[t] + pz[64 + t], kkt = pk[t] + pk[64 + t], qdt = pq[t] + pq[64 + t];
        const float gm = g_s[t];
        const float dbt = (pyv[t] + pyv[64 + t]) + gm * zkt + (ppb[t] + ppb[64 + t]);
        float dgam = b_s[t] * zkt + qdt;
        if (t == FP_C - 1) dgam += ((fr[0] + fr[1]) + (fr[2] + fr[3])) + ((fr[4] + fr[5]) + (fr[6] + fr[7]));
        // s(m) = sum_{t >= m} Gamma[t][m] dgamma_t = dgamma_m + alpha_{m+1} s(m+1): a suffix affine scan
        float sb = dgam, sa = lane + 1 < FP_C ? a_s[lane + 1] : 0.0f;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float bn = __shfl_down(sb, o), an = __shfl_down(sa, o);
            if (lane + o < 64) {
                sb = fmaf(sa, bn, sb);
                sa *= an;
            }
        }
        // row C-1's K.dKt term of dGamma: e(m) = sum_{i < m} (K.dKt)_i Gamma[m-1][i],
        // e(m+1) = alpha_m e(m) + (K.dKt)_m, weighted by Gamma[C-1][m]
        float eb = kkt, ea = a_s[t];
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float bp = __shfl_up(eb, o), ap = __shfl_up(ea, o);
            if (lane >= o) {
                eb = fmaf(ea, bp, eb);
                ea *= ap;
            }
        }
        float em = __shfl_up(eb, 1);
        if (lane == 0) em = 0.0f;
        const float gprev = lane ? g_s[lane - 1] : 1.0f;   // gamma_{m-1}
        if (t < valid) {
            const long gi = ((long)b * T + t0 + t) * H + h;
            dalpha[gi] = fmaf(gprev, sb, fmaf(gt_s[t], em, dlr[t]));
            dbeta[gi] = dbt;
        }
    }
}

// ---------------------------------------------------------------- outputs and E
// O = Qp S + M Uv for one chunk (C = 64, dh = 128), written token-major.  256
// threads, 51 KB of LDS (three blocks per CU).
constexpr int FO_NT = 256;
constexpr int FO_LDS_F = FP_C * FP_LC + FP_C * FP_LK;
static_assert(FO_LDS_F * 4 <= 65536, "LDS of the output kernel");

__global__ __launch_bounds__(FO_NT) void ck_out_fused_k(int T, int H, int NC, ChunkWs w, float* __restrict__ o) {
    extern __shared__ float4 fo_lds4[];
    float* const QM = reinterpret_cast<float*>(fo_lds4);  // Qp k-half, then M   [64][68]
    float* const SU = QM + FP_C * FP_LC;                   // S k-half, then Uv   [64][132]
    const long n = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int li = lane & 15, l4 = lane >> 4;
    const long u = n / NC;
    const int c = (int)(n - u * NC);
    const int b = (int)(u / H), h = (int)(u - (long)b * H);
    const int t0 = c * FP_C;
    const int valid = min(FP_C, T - t0);
    const long cd = n * FP_C * FP_D, cc = n * FP_C * FP_C, dd = n * FP_D * FP_D;
    const int m0 = 32 * (wv >> 1), n0 = 64 * (wv & 1);
    f32x4 acc[2][4];
    acc_zero(acc);
#pragma unroll
    for (int ph = 0; ph < 3; ++ph) {
        const float* a_src = ph < 2 ? w.Qp + cd + 64 * ph : w.Mm + cc;
        const int a_ld = ph < 2 ? FP_D : FP_C;
        const float* b_src = ph < 2 ? w.S + dd + 64 * ph * FP_D : w.Uv + cd;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = tid + i * FO_NT, r = e >> 4, f = 4 * (e & 15);
            *reinterpret_cast<float4*>(QM + r * FP_LC + f) = *reinterpret_cast<const float4*>(a_src + r * a_ld + f);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = tid + i * FO_NT, r = e >> 5, f = 4 * (e & 31);
            *reinterpret_cast<float4*>(SU + r * FP_LK + f) = *reinterpret_cast<const float4*>(b_src + r * FP_D + f);
        }
        __syncthreads();
        wave_mm<2, 4, true, false, false, false>(acc, 0, 64, QM, FP_LC, nullptr, SU, FP_LK, nullptr, m0, n0, lane);
        __syncthreads();
    }
    const long rowbase = ((long)b * T + t0) * H * FP_D + (long)h * FP_D;
    const long rowstride = (long)H * FP_D;
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = m0 + 16 * x + 4 * l4 + r, f = n0 + 16 * y + li;
                if (t < valid) o[rowbase + (long)t * rowstride + f] = acc[x][y][r];
            }
}


// Forward state scan of the fused C = 64, dh = 128 path, from the per-chunk
// factors instead of G' = gamma_C I - Kt^T W and H = Kt^T Uv
// (Kt = diag(Gamma[C-1,:]) K):
//   X_0 = 0,  X_{c+1} = gamma_C X_c + Kt^T (Uv - W X_c)
// It also stores U_c = Uv - W X_c of every chunk (the last included) for the
// backward.
// One block per (unit, 64-column half), 8 waves; per chunk two dependent
// products, 64 x 64 x 128 (Z) and 128 x 64 x 64 (the update).  W and Kt of the
// next chunk (and Uv or E at this lane's outputs) are prefetched into
// registers during the products.  LDS: W, Kt [64][132], X^T [64][132], Z [64][68].
constexpr int S2_LDS_F = 3 * FP_C * FP_LK + FP_C * FP_LC;

__global__ __launch_bounds__(FP_NT) void ck_scan2_k(ChunkWs w, const uint16_t* __restrict__ kin, int T, int H,
                                                    float* __restrict__ X, int NC) {
    extern __shared__ float4 s2_lds4[];
    float* const Ws = reinterpret_cast<float*>(s2_lds4);  // W_c   [t][a]
    float* const Ks = Ws + FP_C * FP_LK;                  // Kt_c  [t][a]
    float* const Xt = Ks + FP_C * FP_LK;                  // X^T   [n][a], this block's 64 columns
    float* const Zs = Xt + FP_C * FP_LK;                  // Z     [t][n]
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int li = lane & 15, l4 = lane >> 4;
    const long u = blockIdx.x >> 1;
    const int col0 = (blockIdx.x & 1) * 64;
    const int ub = (int)(u / H), uh = (int)(u - (long)ub * H);
    const long DD = (long)FP_D * FP_D, CD = (long)FP_C * FP_D;
    float* const Xu = X + u * NC * DD;
    const int m1 = 16 * (wv >> 1), n1 = 32 * (wv & 1);  // step 1 tile: t x n
    const int m2 = 32 * (wv >> 1), n2 = 32 * (wv & 1);  // step 2 tile: a x n
    const float* const A1s = Ws;
    const float* const A2s = Ks;

    // the starting slot is zero
    const int c_first = 0;
    for (int e = tid; e < 64 * FP_D; e += FP_NT) {
        const int nn = e & 63, a = e >> 6;
        Xt[nn * FP_LK + a] = 0.0f;
        Xu[(long)c_first * DD + (long)a * FP_D + col0 + nn] = 0.0f;
    }

    // chunk n's W, K rows and Gamma[C-1, :] of this thread, gamma_C and Uv at
    // this lane's step-1 outputs, held in named registers (arrays carried
    // across the chunk loop go to scratch)
    float4 w0, w1, w2, w3;
    uint2 k0, k1, k2, k3;  // 4 bf16 each
    float g0, g1, g2, g3, gC = 0.0f;
    float r1[2][4];
#define S2_ROW(i) ((tid + (i) * FP_NT) >> 5)
#define S2_COL(i) (4 * ((tid + (i) * FP_NT) & 31))
#define S2_LDK(dst, i)                                                                                 \
    do {                                                                                               \
        const int t_ = S2_ROW(i);                                                                      \
        dst = make_uint2(0u, 0u);                                                                      \
        if (t_ < valid_)                                                                               \
            dst = *reinterpret_cast<const uint2*>(kin + ((long)(ub * T + t0_ + t_) * H + uh) * FP_D +  \
                                                  S2_COL(i));                                          \
    } while (0)
#define S2_STAGE(cc)                                                                                   \
    do {                                                                                               \
        const long n_ = u * NC + (cc);                                                                 \
        const int t0_ = (cc) * FP_C, valid_ = min(FP_C, T - t0_);                                      \
        const float* W_ = w.W + n_ * CD;                                                               \
        w0 = *reinterpret_cast<const float4*>(W_ + S2_ROW(0) * FP_D + S2_COL(0));                      \
        w1 = *reinterpret_cast<const float4*>(W_ + S2_ROW(1) * FP_D + S2_COL(1));                      \
        w2 = *reinterpret_cast<const float4*>(W_ + S2_ROW(2) * FP_D + S2_COL(2));                      \
        w3 = *reinterpret_cast<const float4*>(W_ + S2_ROW(3) * FP_D + S2_COL(3));                      \
        S2_LDK(k0, 0);                                                                                 \
        S2_LDK(k1, 1);                                                                                 \
        S2_LDK(k2, 2);                                                                                 \
        S2_LDK(k3, 3);                                                                                 \
        g0 = w.gt[n_ * FP_C + S2_ROW(0)];                                                              \
        g1 = w.gt[n_ * FP_C + S2_ROW(1)];                                                              \
        g2 = w.gt[n_ * FP_C + S2_ROW(2)];                                                              \
        g3 = w.gt[n_ * FP_C + S2_ROW(3)];                                                              \
        gC = w.gC[n_];                                                                                 \
        _Pragma("unroll") for (int y = 0; y < 2; ++y) _Pragma("unroll") for (int r = 0; r < 4; ++r)     \
            r1[y][r] = w.Uv[n_ * CD + (m1 + 4 * l4 + r) * FP_D + col0 + n1 + 16 * y + li];             \
    } while (0)
#define S2_PUT(i, wi, ki, gi)                                                                          \
    do {                                                                                               \
        *reinterpret_cast<float4*>(Ws + S2_ROW(i) * FP_LK + S2_COL(i)) = (wi);                         \
        *reinterpret_cast<float4*>(Ks + S2_ROW(i) * FP_LK + S2_COL(i)) =                               \
            make_float4((gi) * __uint_as_float((ki).x << 16), (gi) * __uint_as_float((ki).x & 0xffff0000u), \
                        (gi) * __uint_as_float((ki).y << 16), (gi) * __uint_as_float((ki).y & 0xffff0000u)); \
    } while (0)
    int c = c_first;
    S2_STAGE(c);
    // step 1 of the last chunk runs too: its U goes to the backward
    for (int s = 0; s < NC; ++s) {
        const int cn = c + 1;  // output slot
        __syncthreads();                     // the previous chunk's readers of Ws, Ks, Zs are done
        S2_PUT(0, w0, k0, g0);
        S2_PUT(1, w1, k1, g1);
        S2_PUT(2, w2, k2, g2);
        S2_PUT(3, w3, k3, g3);
        const float gCc = gC;
        float z1[2][4];
#pragma unroll
        for (int y = 0; y < 2; ++y)
#pragma unroll
            for (int r = 0; r < 4; ++r) z1[y][r] = r1[y][r];
        __syncthreads();  // Ws, Ks and X^T ready
        if (s + 1 < NC) S2_STAGE(cn);
        // step 1: Z = U = Uv - W X
        {
            f32x4 acc[1][2];
            acc_zero(acc);
            wave_mm<1, 2, true, false, true, false>(acc, 0, FP_D, A1s, FP_LK, nullptr, Xt, FP_LK, nullptr, m1, n1,
                                                    lane);
            float* const Ug = w.Uu + (u * NC + c) * CD;
#pragma unroll
            for (int y = 0; y < 2; ++y)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = m1 + 4 * l4 + r, nn = n1 + 16 * y + li;
                    const float z = z1[y][r] - acc[0][y][r];
                    Zs[t * FP_LC + nn] = z;
                    Ug[t * FP_D + col0 + nn] = z;  // U = Uv - W S of chunk c
                }
        }
        if (s == NC - 1) break;
        __syncthreads();  // Z ready
        // step 2: X' = gamma_C X + Kt^T Z; each wave reads and then overwrites
        // only its own elements of X^T
        {
            f32x4 acc[2][2];
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int y = 0; y < 2; ++y)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float xv = Xt[(n2 + 16 * y + li) * FP_LK + m2 + 16 * x + 4 * l4 + r];
                        acc[x][y][r] = gCc * xv;
                    }
            wave_mm<2, 2, false, false, false, false>(acc, 0, FP_C, A2s, FP_LK, nullptr, Zs, FP_LC, nullptr, m2, n2,
                                                      lane);
            float* const Xn = Xu + (long)cn * DD;
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int y = 0; y < 2; ++y)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int a = m2 + 16 * x + 4 * l4 + r, nn = n2 + 16 * y + li;
                        Xt[nn * FP_LK + a] = acc[x][y][r];
                        Xn[(long)a * FP_D + col0 + nn] = acc[x][y][r];
                    }
        }
        c = cn;
    }
#undef S2_ROW
#undef S2_COL
#undef S2_STAGE
#undef S2_LDK
#undef S2_PUT
}

// Reverse scan of the fused path with E_c = Qp_c^T dO_c formed in place:
//   X_{NC-1} = 0,  X_{c-1} = gamma_C X_c + Qp_c^T dO_c - W_c^T diag(Gamma[C-1,:]) K_c X_c
// E is the same 128 x 64 x 64 shape as the update product, so it goes into
// the same accumulators.  K is staged as bf16 (exact: a bf16 input) and
// Gamma[C-1, :] is applied to the rows of K X; the block's 64 columns of dO
// come straight from the bf16 input (zero past T).  LDS: W, Qp, X^T f32
// [64][132], Z [64][68], K bf16 [64][136], dO bf16 [64][72], Gamma[C-1, :].
constexpr int S3_LB = 64 + 8;
constexpr int S3_LDS_F = 3 * FP_C * FP_LK + FP_C * FP_LC + FP_C * FB_LB / 2 + FP_C * S3_LB / 2 + FP_C;

__global__ __launch_bounds__(FP_NT) void ck_scan2_bwd_k(ChunkWs w, const uint16_t* __restrict__ kin,
                                                        const uint16_t* __restrict__ d_o, int T, int H, int NC) {
    extern __shared__ float4 s3_lds4[];
    float* const Ws = reinterpret_cast<float*>(s3_lds4);                // W_c   [t][a]
    float* const Qs = Ws + FP_C * FP_LK;                                // Qp_c  [t][a]
    float* const Xt = Qs + FP_C * FP_LK;                                // X^T   [n][a]
    float* const Zs = Xt + FP_C * FP_LK;                                // Z     [t][n]
    uint16_t* const Kb = reinterpret_cast<uint16_t*>(Zs + FP_C * FP_LC);  // K_c   [t][a]
    uint16_t* const Ob = Kb + FP_C * FB_LB;                             // dO_c  [t][n]
    float* const gts = reinterpret_cast<float*>(Ob + FP_C * S3_LB);     // Gamma[C-1, :]
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int li = lane & 15, l4 = lane >> 4;
    const long u = blockIdx.x >> 1;
    const int col0 = (blockIdx.x & 1) * 64;
    const int b = (int)(u / H), h = (int)(u - (long)b * H);
    const long DD = (long)FP_D * FP_D, CD = (long)FP_C * FP_D;
    float* const Xu = w.dSp + u * NC * DD;
    const int m1 = 16 * (wv >> 1), n1 = 32 * (wv & 1);  // step 1 tile: t x n
    const int m2 = 32 * (wv >> 1), n2 = 32 * (wv & 1);  // step 2 tile: a x n

    for (int e = tid; e < 64 * FP_D; e += FP_NT) {
        const int nn = e & 63, a = e >> 6;
        Xt[nn * FP_LK + a] = 0.0f;
        Xu[(long)(NC - 1) * DD + (long)a * FP_D + col0 + nn] = 0.0f;
    }
    if (NC < 2) return;

    // chunk c's W, Qp, K rows of this thread, its two quarter-rows of dO,
    // Gamma[C-1, :] (first wave) and gamma_C, in named registers
    float4 w0, w1, w2, w3, q0, q1, q2, q3;
    uint2 k0, k1, k2, k3, o0, o1;
    float gtv = 0.0f, gC = 0.0f;
#define S3_ROW(i) ((tid + (i) * FP_NT) >> 5)
#define S3_COL(i) (4 * ((tid + (i) * FP_NT) & 31))
#define S3_OROW(i) ((tid + (i) * FP_NT) >> 4)
#define S3_OCOL(i) (4 * ((tid + (i) * FP_NT) & 15))
#define S3_LD4(dst, base, i) dst = *reinterpret_cast<const float4*>((base) + S3_ROW(i) * FP_D + S3_COL(i))
#define S3_LDO(dst, i)                                                                                    \
    do {                                                                                                  \
        const int t_ = S3_OROW(i);                                                                        \
        dst = make_uint2(0u, 0u);                                                                         \
        if (t_ < valid_)                                                                                  \
            dst = *reinterpret_cast<const uint2*>(d_o + ((long)(b * T + t0_ + t_) * H + h) * FP_D + col0 + \
                                                  S3_OCOL(i));                                            \
    } while (0)
#define S3_LDK(dst, i)                                                                                    \
    do {                                                                                                  \
        const int t_ = S3_ROW(i);                                                                         \
        dst = make_uint2(0u, 0u);                                                                         \
        if (t_ < valid_)                                                                                  \
            dst = *reinterpret_cast<const uint2*>(kin + ((long)(b * T + t0_ + t_) * H + h) * FP_D + S3_COL(i)); \
    } while (0)
#define S3_STAGE(cc)                                                                   \
    do {                                                                               \
        const long n_ = u * NC + (cc);                                                 \
        const int t0_ = (cc) * FP_C, valid_ = min(FP_C, T - t0_);                      \
        S3_LD4(w0, w.W + n_ * CD, 0);                                                  \
        S3_LD4(w1, w.W + n_ * CD, 1);                                                  \
        S3_LD4(w2, w.W + n_ * CD, 2);                                                  \
        S3_LD4(w3, w.W + n_ * CD, 3);                                                  \
        S3_LD4(q0, w.Qp + n_ * CD, 0);                                                 \
        S3_LD4(q1, w.Qp + n_ * CD, 1);                                                 \
        S3_LD4(q2, w.Qp + n_ * CD, 2);                                                 \
        S3_LD4(q3, w.Qp + n_ * CD, 3);                                                 \
        S3_LDK(k0, 0);                                                                 \
        S3_LDK(k1, 1);                                                                 \
        S3_LDK(k2, 2);                                                                 \
        S3_LDK(k3, 3);                                                                 \
        S3_LDO(o0, 0);                                                                 \
        S3_LDO(o1, 1);                                                                 \
        if (tid < FP_C) gtv = w.gt[n_ * FP_C + tid];                                   \
        gC = w.gC[n_];                                                                 \
    } while (0)
#define S3_PUT(i, wi, qi, ki)                                                                                  \
    do {                                                                                                       \
        *reinterpret_cast<float4*>(Ws + S3_ROW(i) * FP_LK + S3_COL(i)) = (wi);                                 \
        *reinterpret_cast<float4*>(Qs + S3_ROW(i) * FP_LK + S3_COL(i)) = (qi);                                 \
        *reinterpret_cast<uint2*>(Kb + S3_ROW(i) * FB_LB + S3_COL(i)) = (ki);                                  \
    } while (0)
    int c = NC - 1;
    S3_STAGE(c);
    for (int s = 0; s < NC - 1; ++s) {
        const int cn = c - 1;  // output slot
        __syncthreads();       // the previous chunk's readers of the staged operands are done
        S3_PUT(0, w0, q0, k0);
        S3_PUT(1, w1, q1, k1);
        S3_PUT(2, w2, q2, k2);
        S3_PUT(3, w3, q3, k3);
        *reinterpret_cast<uint2*>(Ob + S3_OROW(0) * S3_LB + S3_OCOL(0)) = o0;
        *reinterpret_cast<uint2*>(Ob + S3_OROW(1) * S3_LB + S3_OCOL(1)) = o1;
        if (tid < FP_C) gts[tid] = gtv;
        const float gCc = gC;
        __syncthreads();  // staged operands and X^T ready
        if (s + 1 < NC - 1) S3_STAGE(cn);
        // step 1: Z = -diag(Gamma[C-1,:]) K X
        {
            f32x4 acc[1][2];
            acc_zero(acc);
            wave_mm<1, 2, true, true, true, false>(acc, 0, FP_D, Kb, FB_LB, nullptr, Xt, FP_LK, nullptr, m1, n1, lane);
#pragma unroll
            for (int y = 0; y < 2; ++y)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = m1 + 4 * l4 + r;
                    Zs[t * FP_LC + n1 + 16 * y + li] = -(gts[t] * acc[0][y][r]);
                }
        }
        __syncthreads();  // Z ready
        // step 2: X' = gamma_C X + Qp^T dO + W^T Z; each wave reads and then
        // overwrites only its own elements of X^T
        {
            f32x4 acc[2][2];
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int y = 0; y < 2; ++y)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[x][y][r] = gCc * Xt[(n2 + 16 * y + li) * FP_LK + m2 + 16 * x + 4 * l4 + r];
            wave_mm<2, 2, false, false, false, true>(acc, 0, FP_C, Qs, FP_LK, nullptr, Ob, S3_LB, nullptr, m2, n2,
                                                     lane);
            wave_mm<2, 2, false, false, false, false>(acc, 0, FP_C, Ws, FP_LK, nullptr, Zs, FP_LC, nullptr, m2, n2,
                                                      lane);
            float* const Xn = Xu + (long)cn * DD;
#pragma unroll
            for (int x = 0; x < 2; ++x)
#pragma unroll
                for (int y = 0; y < 2; ++y)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int a = m2 + 16 * x + 4 * l4 + r, nn = n2 + 16 * y + li;
                        Xt[nn * FP_LK + a] = acc[x][y][r];
                        Xn[(long)a * FP_D + col0 + nn] = acc[x][y][r];
                    }
        }
        c = cn;
    }
#undef S3_ROW
#undef S3_COL
#undef S3_OROW
#undef S3_OCOL
#undef S3_LD4
#undef S3_LDO
#undef S3_STAGE
#undef S3_LDK
#undef S3_PUT
}

// The state scan over chunks: the persistent kernel for dh = 128, else one
// batched GEMM launch per chunk.
static int scan(bool tr, const ChunkDims& d, const float* Gp, const float* R, float* X, hipStream_t st) {
    const long us = (long)d.NC * d.DD;
    if (d.dh == SC_D) {
        constexpr size_t lds = (size_t)(SC_D + 64) * SC_LD * sizeof(float);
        const void* fn = tr ? reinterpret_cast<const void*>(&ck_scan_k<true>)
                            : reinterpret_cast<const void*>(&ck_scan_k<false>);
        if (int arc = allow_lds(fn, lds)) return arc;
        int rc = pre_launch("chunk_scan");
        if (rc) return rc;
        if (tr)
            hipLaunchKernelGGL(ck_scan_k<true>, dim3((unsigned)(2 * d.U)), dim3(SC_NT), lds, st, Gp, R, X, d.NC);
        else
            hipLaunchKernelGGL(ck_scan_k<false>, dim3((unsigned)(2 * d.U)), dim3(SC_NT), lds, st, Gp, R, X, d.NC);
        return post_launch("chunk_scan");
    }
    const int first = tr ? d.NC - 1 : 0;
    CK_LAUNCH("chunk_zero", ck_zero_slot_k, dim3(nblk(d.U * d.DD)), dim3(256), X, us, (long)first * d.DD, d.DD,
              d.U * d.DD);
    for (int s = 0; s + 1 < d.NC; ++s) {
        const int c = tr ? d.NC - 1 - s : s;
        const long oc = (long)c * d.DD;
        float* out = X + (tr ? oc - d.DD : oc + d.DD);
        int rc = bgemm(tr ? 1 : 0, 0, d.dh, d.dh, d.dh, 1.f, Gp + oc, d.dh, us, X + oc, d.dh, us, 0.f, out, d.dh, us,
                       R + oc, us, d.U, st, "chunk_scan");
        if (rc) return rc;
    }
    return ASCA_OK;
}

// The factorised forward state scan of the fused C = 64, dh = 128 path.
static int scan2(const ChunkDims& d, const ChunkWs& w, const uint16_t* k, hipStream_t st) {
    constexpr size_t lds = (size_t)S2_LDS_F * sizeof(float);
    if (int arc = allow_lds(reinterpret_cast<const void*>(&ck_scan2_k), lds)) return arc;
    int rc = pre_launch("chunk_scan2");
    if (rc) return rc;
    hipLaunchKernelGGL(ck_scan2_k, dim3((unsigned)(2 * d.U)), dim3(FP_NT), lds, st, w, k, d.T, d.H, w.S, d.NC);
    return post_launch("chunk_scan2");
}

// The state scan and the outputs O = Qp S + M Uv.
static int chunk_fwd_tail(const ChunkDims& d, const ChunkWs& w, const uint16_t* k, float* o, hipStream_t st,
                          bool fused) {
    const int C = d.C, dh = d.dh;
    int rc;
    if (fused) {
        if ((rc = scan2(d, w, k, st))) return rc;
        CK_LAUNCH_LDS("chunk_out_fused", ck_out_fused_k, dim3((unsigned)d.N), dim3(FO_NT),
                  (size_t)FO_LDS_F * sizeof(float), d.T, d.H, d.NC, w, o);
        return ASCA_OK;
    }
    // state scan over chunks: S_0 = 0, S_{c+1} = G'_c S_c + H_c
    if ((rc = scan(false, d, w.Gp, w.H, w.S, st))) return rc;
    if ((rc = bgemm(0, 0, C, dh, dh, 1.f, w.Qp, dh, d.CD, w.S, dh, d.DD, 0.f, w.Ou, dh, d.CD, nullptr, 0, d.N, st,
                    "chunk_O1")) ||
        (rc = bgemm(0, 0, C, dh, C, 1.f, w.Mm, C, d.CC, w.Uv, dh, d.CD, 1.f, w.Ou, dh, d.CD, nullptr, 0, d.N, st,
                    "chunk_O2")))
        return rc;
    const int tot_out4 = (int)((long)d.B * d.T * d.H * dh / 4);
    CK_LAUNCH("chunk_out", ck_out_k, dim3(nblk(tot_out4)), dim3(256), w.Ou, o, d.T, d.H, dh, d.Tp, tot_out4);
    return ASCA_OK;
}

}  // namespace asca

using namespace asca;

static int chunk_fwd_decomposed(const ChunkDims& d, const ChunkWs& w, const float* alpha, const float* beta,
                                float* o, hipStream_t st);
static int chunk_bwd_decomposed(const ChunkDims& d, const ChunkWs& w, float* dq, float* dk, float* dv,
                                float* dalpha, float* dbeta, hipStream_t st);

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
    if (C == FP_C && dh == FP_D) {
        // one fused kernel for every state-independent part of every chunk
        constexpr size_t lds = (size_t)FP_LDS_F * sizeof(float);
        if (int arc = allow_lds(reinterpret_cast<const void*>(&ck_fwd_prep_k), lds)) return arc;
        rc = pre_launch("chunk_fwd_prep");
        if (rc) return rc;
        hipLaunchKernelGGL(ck_fwd_prep_k, dim3((unsigned)d.N), dim3(FP_NT), lds, st, q, k, v, alpha, beta, T, H,
                           d.NC, w);
        if ((rc = post_launch("chunk_fwd_prep"))) return rc;
        return chunk_fwd_tail(d, w, k, o, st, true);
    }
    const int tot_in4 = (int)(d.U * d.Tp * dh / 4);
    CK_LAUNCH("chunk_in", ck_in_k, dim3(nblk(tot_in4)), dim3(256), q, w.Qu, T, H, dh, d.Tp, tot_in4);
    CK_LAUNCH("chunk_in", ck_in_k, dim3(nblk(tot_in4)), dim3(256), k, w.Ku, T, H, dh, d.Tp, tot_in4);
    CK_LAUNCH("chunk_in", ck_in_k, dim3(nblk(tot_in4)), dim3(256), v, w.Vu, T, H, dh, d.Tp, tot_in4);
    return chunk_fwd_decomposed(d, w, alpha, beta, o, st);
}

}  // extern "C"

// The decomposed forward from the unit-major f32 copies of q, k, v in the
// workspace (Qu, Ku, Vu): every per-chunk product a batched GEMM.
static int chunk_fwd_decomposed(const ChunkDims& d, const ChunkWs& w, const float* alpha, const float* beta,
                                float* o, hipStream_t st) {
    const int T = d.T, H = d.H, dh = d.dh, C = d.C;
    int rc;
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
    CK_LAUNCH("chunk_tri", ck_tri_k, dim3((unsigned)d.N), dim3(256), w.Am, w.Bm, w.Gam, w.be, C, w.Tm, w.Mm);
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
    return chunk_fwd_tail(d, w, nullptr, o, st, false);
}

extern "C" {

int asca_chunk_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* d_o, void* ws, float* dq,
                   float* dk, float* dv, float* dalpha, float* dbeta, int B, int T, int H, int dh, int C,
                   void* stream) {
    int rc = chunk_check(B, T, H, dh, C);
    if (rc) return rc;
    if ((long)B * T * H == 0) return ASCA_OK;
    if (!q || !k || !v || !d_o || !ws || !dq || !dk || !dv || !dalpha || !dbeta)
        return fail(ASCA_ERR_INVALID, "asca_chunk_bwd: null pointer");
    const ChunkDims d = chunk_dims(B, T, H, dh, C);
    const ChunkWs w = chunk_ws(d, reinterpret_cast<float*>(ws));
    const hipStream_t st = as_stream(stream);
    if (C == FP_C && dh == FP_D) {
        // E, the reverse scan, then one fused kernel for all per-chunk gradients
        {
            constexpr size_t lds = (size_t)S3_LDS_F * sizeof(float);
            if (int arc = allow_lds(reinterpret_cast<const void*>(&ck_scan2_bwd_k), lds)) return arc;
            if ((rc = pre_launch("chunk_scan2_bwd"))) return rc;
            hipLaunchKernelGGL(ck_scan2_bwd_k, dim3((unsigned)(2 * d.U)), dim3(FP_NT), lds, st, w, k, d_o, T, H,
                               d.NC);
            if ((rc = post_launch("chunk_scan2_bwd"))) return rc;
        }
        constexpr size_t lds = (size_t)FB_LDS_F * sizeof(float);
        if (int arc = allow_lds(reinterpret_cast<const void*>(&ck_bwd_fused_k), lds)) return arc;
        if ((rc = pre_launch("chunk_bwd_fused"))) return rc;
        hipLaunchKernelGGL(ck_bwd_fused_k, dim3((unsigned)d.N), dim3(FP_NT), lds, st, q, k, v, d_o, T, H, d.NC, w,
                           dq, dk, dv, dalpha, dbeta);
        return post_launch("chunk_bwd_fused");
    }
    const int tot_in4 = (int)(d.U * d.Tp * dh / 4);
    CK_LAUNCH("chunk_in", ck_in_k, dim3(nblk(tot_in4)), dim3(256), d_o, w.dOu, T, H, dh, d.Tp, tot_in4);
    return chunk_bwd_decomposed(d, w, dq, dk, dv, dalpha, dbeta, st);
}

}  // extern "C"

// The decomposed backward from the forward's workspace and the unit-major f32
// copy of dO (dOu).
static int chunk_bwd_decomposed(const ChunkDims& d, const ChunkWs& w, float* dq, float* dk, float* dv,
                                float* dalpha, float* dbeta, hipStream_t st) {
    const int B = d.B, T = d.T, H = d.H, dh = d.dh, C = d.C;
    const int tot_in4 = (int)(d.U * d.Tp * dh / 4);
    int rc;
    CK_LAUNCH("chunk_rowscale", ck_rowscale_k, dim3(nblk(tot_in4)), dim3(256), w.dOu, w.gam, w.dOg, dh, tot_in4);
    // E_c = Qp^T dO_c; reverse scan dS'_{c-1} = G'_c^T dS'_c + E_c, dS'_{NC-1} = 0
    if ((rc = bgemm(1, 0, dh, dh, C, 1.f, w.Qp, dh, d.CD, w.dOu, dh, d.CD, 0.f, w.E, dh, d.DD, nullptr, 0, d.N, st,
                    "chunk_E")))
        return rc;
    if ((rc = scan(true, d, w.Gp, w.E, w.dSp, st))) return rc;
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
    const int tot_out4 = (int)((long)B * T * H * dh / 4);
    CK_LAUNCH("chunk_bwd_out", ck_bwd_out_k, dim3(nblk(tot_out4)), dim3(256), w.dqu, w.dku, w.Z, w.dKt, w.Y, w.be,
              w.gam, w.gt, T, H, dh, d.Tp, dq, dk, dv, tot_out4);
    const long tot_g = (long)B * T * H;
    CK_LAUNCH("chunk_gates_out", ck_gates_out_k, dim3(nblk(tot_g)), dim3(256), w.dal, w.dbe, T, H, d.Tp, dalpha, dbeta,
              tot_g);
    return ASCA_OK;
}

extern "C" {

int asca_chunk_ws_bytes_f32(int B, int T, int H, int dh, int C, size_t* bytes) {
    if (!bytes) return fail(ASCA_ERR_INVALID, "null output pointer");
    int rc = chunk_check(B, T, H, dh, C);
    if (rc) return rc;
    *bytes = chunk_ws(chunk_dims(B, T, H, dh, C), nullptr, false).total * sizeof(float);
    return ASCA_OK;
}

static int chunk_in_f32(const float* src, float* dst, const ChunkDims& d, hipStream_t st) {
    const int tot_in4 = (int)(d.U * d.Tp * d.dh / 4);
    if ((reinterpret_cast<uintptr_t>(src) & 15) == 0)
        CK_LAUNCH("chunk_in_f32", ck_in_f32_k<true>, dim3(nblk(tot_in4)), dim3(256), src, dst, d.T, d.H, d.dh, d.Tp,
                  tot_in4);
    else
        CK_LAUNCH("chunk_in_f32", ck_in_f32_k<false>, dim3(nblk(tot_in4)), dim3(256), src, dst, d.T, d.H, d.dh, d.Tp,
                  tot_in4);
    return ASCA_OK;
}

int asca_chunk_fwd_f32(const float* q, const float* k, const float* v, const float* alpha, const float* beta,
                       float* o, void* ws, int B, int T, int H, int dh, int C, void* stream) {
    int rc = chunk_check(B, T, H, dh, C);
    if (rc) return rc;
    if ((long)B * T * H == 0) return ASCA_OK;
    if (!q || !k || !v || !alpha || !beta || !o || !ws)
        return fail(ASCA_ERR_INVALID, "asca_chunk_fwd_f32: null pointer");
    const ChunkDims d = chunk_dims(B, T, H, dh, C);
    const ChunkWs w = chunk_ws(d, reinterpret_cast<float*>(ws), false);
    const hipStream_t st = as_stream(stream);
    if ((rc = chunk_in_f32(q, w.Qu, d, st)) || (rc = chunk_in_f32(k, w.Ku, d, st)) ||
        (rc = chunk_in_f32(v, w.Vu, d, st)))
        return rc;
    return chunk_fwd_decomposed(d, w, alpha, beta, o, st);
}

int asca_chunk_bwd_f32(const float* d_o, void* ws, float* dq, float* dk, float* dv, float* dalpha, float* dbeta,
                       int B, int T, int H, int dh, int C, void* stream) {
    int rc = chunk_check(B, T, H, dh, C);
    if (rc) return rc;
    if ((long)B * T * H == 0) return ASCA_OK;
    if (!d_o || !ws || !dq || !dk || !dv || !dalpha || !dbeta)
        return fail(ASCA_ERR_INVALID, "asca_chunk_bwd_f32: null pointer");
    const ChunkDims d = chunk_dims(B, T, H, dh, C);
    const ChunkWs w = chunk_ws(d, reinterpret_cast<float*>(ws), false);
    const hipStream_t st = as_stream(stream);
    if ((rc = chunk_in_f32(d_o, w.dOu, d, st))) return rc;
    return chunk_bwd_decomposed(d, w, dq, dk, dv, dalpha, dbeta, st);
}

}  // extern "C"
