// Device-resident training step of the ASCA model: Model::forward,
// Model::backward and the AdamW step over every parameter
// (rust/src/model.rs:528-802, rust/src/train.rs:176-186), with DeltaBlock
// forward/backward (rust/src/delta.rs:121-207,615-674) and HashMoe
// (model.rs:187-306,339-497) as in the reference, but with weights, gradients,
// AdamW moments and activations resident in HBM for the whole step and every
// dense product on the MFMA GEMM.
//
// Structure per layer (model.rs:665-678): x_mid = x + Delta(x) (the delta block
// takes the raw residual stream), x_out = x_mid + MoE(RMSNorm(x_mid)); then
// h = RMSNorm(x_L), logits = h W_head, softmax cross-entropy against targets.
// The backward mirrors model.rs:729-794, and AdamW::update runs per parameter
// tensor with its per-tensor step counter (tensor.rs:392-453), bit-exact.
//
// Parameters live in one flat f32 buffer (and gradients, m, v in three more),
// tensors in the reference's params() order: embed, head, then per layer
// w_qkv, b_qkv, w_gate, b_gate, w_o, b_o, w1, b1, w2, b2 (model.rs:596-603,
// delta.rs:96-105, model.rs:103-105).
#include <algorithm>
#include <cstdio>
#include <string>
#include <type_traits>
#include <vector>

#include "common.h"
#include "gemm.h"
#include "moe.h"
#include "ops.h"
#include "runtime.h"

namespace asca {

constexpr float MODEL_EPS = 1e-6f;  // model.rs:14

// q, k, v split out of the projection rows, q and k L2-normalised per head
// (x / max(|x|, 1e-8)) with the norms kept, and alpha, beta = sigmoid of the
// gate logits (delta.rs:131-186, tensor.rs:245-248).  One block per row.
__global__ __launch_bounds__(256) void qkv_prep_k(const float* __restrict__ qkv, const float* __restrict__ gate,
                                                  int H, int dh, float* __restrict__ q, float* __restrict__ k,
                                                  float* __restrict__ v, float* __restrict__ qn,
                                                  float* __restrict__ kn, float* __restrict__ alpha,
                                                  float* __restrict__ beta) {
    const long r = blockIdx.x;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int d = H * dh;
    const float* src = qkv + r * 3 * d;
    // dh <= 128: two elements per lane; every load of a head is issued before
    // its reductions (clamped indices, unconditional), then the stores
    for (int h = w; h < H; h += 4) {
        float xq[2], xk[2], xv[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int j = min(lane + 64 * e, dh - 1);
            xq[e] = src[h * dh + j];
            xk[e] = src[d + h * dh + j];
            xv[e] = src[2 * d + h * dh + j];
        }
        const float ga = gate[r * 2 * H + h], gb = gate[r * 2 * H + H + h];
        float sq = 0.0f, sk = 0.0f;
#pragma unroll
        for (int e = 0; e < 2; ++e)
            if (lane + 64 * e < dh) {
                sq += xq[e] * xq[e];
                sk += xk[e] * xk[e];
            }
        sq = wave_sum(sq);
        sk = wave_sum(sk);
        const float nq = fmaxf(sqrtf(sq), 1e-8f), nk = fmaxf(sqrtf(sk), 1e-8f);
        const long o = r * d + h * dh;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int j = lane + 64 * e;
            if (j < dh) {
                q[o + j] = xq[e] / nq;
                k[o + j] = xk[e] / nk;
                v[o + j] = xv[e];
            }
        }
        if (lane == 0) {
            qn[r * H + h] = nq;
            kn[r * H + h] = nk;
            alpha[r * H + h] = 1.0f / (1.0f + expf(-ga));
            beta[r * H + h] = 1.0f / (1.0f + expf(-gb));
        }
    }
}

// x0[t] = embed[id_t] (model.rs:655-661).  Ids >= V wrap (memory safety).
__global__ __launch_bounds__(256) void embed_k(const float* __restrict__ embed, const uint32_t* __restrict__ ids,
                                               long T, int d, int V, float* __restrict__ x) {
    const long t = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= T) return;
    const float* src = embed + (long)(ids[t] % (uint32_t)V) * d;
    for (int c = lane; c < d; c += 64) x[t * d + c] = src[c];
}

// Embedding gradient: row v = sum of dx[t] over the tokens with id v, in
// ascending t, starting from zero (model.rs:782-789 after zero_grads).
__global__ __launch_bounds__(256) void embed_grad_k(const float* __restrict__ dx, const int32_t* __restrict__ perm,
                                                    const int32_t* __restrict__ off, int d,
                                                    float* __restrict__ g) {
    const int vrow = blockIdx.x;
    const int lo = off[vrow], hi = off[vrow + 1];
    for (int c = threadIdx.x; c < d; c += 256) {
        float acc = 0.0f;
        for (int i = lo; i < hi; ++i) acc += dx[(long)perm[i] * d + c];
        g[(long)vrow * d + c] = acc;
    }
}

// Mean loss = (sum of per-row losses) / T, one block, fixed order.
__global__ __launch_bounds__(256) void loss_mean_k(const float* __restrict__ losses, long T, float inv_t,
                                                   float* __restrict__ out) {
    __shared__ float part[4];
    float s = 0.0f;
    for (long i = threadIdx.x; i < T; i += 256) s += losses[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) out[0] = (part[0] + part[1] + part[2] + part[3]) * inv_t;
}

// AdamW over all tensors in one launch: block b updates chunk b of tensor j
// with the scalars of step base + j + 1 (the reference increments its step
// counter once per parameter tensor, tensor.rs:393).  Scalars are computed
// per block with the host's f32 operation sequence (binary-exponentiation
// powi, correctly rounded sqrt and division, no contraction), so every
// element update is bit-identical to AdamW::update's CPU body.
struct AdamChunk {
    int tensor;
    int pad;
    long start;
    long len;
};

ASCA_DEV float powi_dev(float a, int b) {
#pragma clang fp contract(off)
    float r = 1.0f;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return r;
}

__global__ __launch_bounds__(256) void adamw_multi_k(float* __restrict__ p, const float* __restrict__ g,
                                                     float* __restrict__ m, float* __restrict__ v,
                                                     const AdamChunk* __restrict__ chunks, uint32_t base, float lr0,
                                                     float b1, float b2, float eps, float wd0) {
#pragma clang fp contract(off)
    const AdamChunk c = chunks[blockIdx.x];
    const int step = (int)(base + (uint32_t)c.tensor + 1u);
    const float bc1 = 1.0f - powi_dev(b1, step);
    const float bc2 = 1.0f - powi_dev(b2, step);
    const float lr = lr0 * sqrtf(bc1 / bc2);
    const float eps_t = eps * sqrtf(bc2);
    const float wd = lr0 * wd0;
    const float omb1 = 1.0f - b1, omb2 = 1.0f - b2;
    auto one = [&](float& pi, float gi, float& mi, float& vi) {
#pragma clang fp contract(off)
        mi = b1 * mi + omb1 * gi;
        vi = b2 * vi + omb2 * gi * gi;
        const float upd = mi / (sqrtf(vi) + eps_t);
        pi -= wd * pi;
        pi -= lr * upd;
    };
    long i0 = c.start;
    if (((c.start | c.len) & 3) == 0) {
        // 16-byte accesses, four float4 of each array in flight per thread
        // (unconditional loads in the unrolled part, the rest one at a time)
        constexpr int U = 4;
        const long n4 = c.len >> 2;
        float4* p4 = reinterpret_cast<float4*>(p + c.start);
        const float4* g4 = reinterpret_cast<const float4*>(g + c.start);
        float4* m4 = reinterpret_cast<float4*>(m + c.start);
        float4* v4 = reinterpret_cast<float4*>(v + c.start);
        long i = threadIdx.x;
        for (; i + 256 * (U - 1) < n4; i += 256 * U) {
            float4 pr[U], gr[U], mr[U], vr[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                gr[u] = g4[i + 256 * u];
                mr[u] = m4[i + 256 * u];
                vr[u] = v4[i + 256 * u];
                pr[u] = p4[i + 256 * u];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                one(pr[u].x, gr[u].x, mr[u].x, vr[u].x);
                one(pr[u].y, gr[u].y, mr[u].y, vr[u].y);
                one(pr[u].z, gr[u].z, mr[u].z, vr[u].z);
                one(pr[u].w, gr[u].w, mr[u].w, vr[u].w);
                m4[i + 256 * u] = mr[u];
                v4[i + 256 * u] = vr[u];
                p4[i + 256 * u] = pr[u];
            }
        }
        for (; i < n4; i += 256) {
            float4 pr = p4[i], gr = g4[i], mr = m4[i], vr = v4[i];
            one(pr.x, gr.x, mr.x, vr.x);
            one(pr.y, gr.y, mr.y, vr.y);
            one(pr.z, gr.z, mr.z, vr.z);
            one(pr.w, gr.w, mr.w, vr.w);
            m4[i] = mr;
            v4[i] = vr;
            p4[i] = pr;
        }
        i0 = c.start + c.len;  // nothing left
    }
    for (long i = i0 + threadIdx.x; i < c.start + c.len; i += 256) {
        float pi = p[i], mi = m[i], vi = v[i];
        one(pi, g[i], mi, vi);
        m[i] = mi;
        v[i] = vi;
        p[i] = pi;
    }
}

struct MTensor {
    std::string name;
    size_t off, n;
    int rows, cols;
};

struct MLayer {
    size_t w_qkv, b_qkv, w_gate, b_gate, w_o, b_o, w1, b1, w2, b2;
};

struct MActs {  // per-layer activations kept for the backward
    float *x_out, *q, *k, *v, *qn, *kn, *al, *be, *o, *x_mid, *xn, *pre, *hid;
    void* dws;
};

struct MDecode {  // decode activations, sized for n sequences
    int n = 0;
    std::vector<void*> allocs;
    float *xa = nullptr, *xb = nullptr, *qkv = nullptr, *gate = nullptr, *o = nullptr, *mid = nullptr,
          *xn = nullptr, *pre = nullptr, *hid = nullptr, *hf = nullptr;
    int32_t *route = nullptr, *perm = nullptr, *off = nullptr;
    void* rws = nullptr;
};

}  // namespace asca

using namespace asca;

struct asca_model {
    int V = 0, d = 0, H = 0, dh = 0, L = 0, E = 0, dff = 0;
    size_t n_params = 0;
    float *p = nullptr, *g = nullptr, *m = nullptr, *v = nullptr;
    std::vector<MTensor> t;
    std::vector<MLayer> lay;
    AdamChunk* chunks = nullptr;
    int n_chunks = 0;
    std::vector<int> chunk0;  // first AdamW chunk of tensor j (size tensors + 1)
    float lr = 3e-4f, b1 = 0.9f, b2 = 0.95f, eps = 1e-8f, wd = 0.01f;
    uint32_t adam_step = 0;
    // activation workspace, sized for one (batch, seq)
    int batch = 0, seq = 0;
    std::vector<void*> allocs;
    std::vector<MActs> acts;
    float *x0 = nullptr, *qkv_t = nullptr, *gate_t = nullptr, *h_final = nullptr, *logits = nullptr;
    float *dlogits = nullptr, *losses = nullptr, *loss = nullptr;
    float *dxn = nullptr, *dtmp = nullptr;
    // two sets, alternating by layer, of the gradients the weight-gradient
    // stream reads while the next layer's backward runs
    float *dx[2] = {nullptr, nullptr}, *dmid[2] = {nullptr, nullptr}, *dqkv[2] = {nullptr, nullptr},
          *dgate[2] = {nullptr, nullptr}, *dpre[2] = {nullptr, nullptr};
    // weight-gradient stream and optimiser stream (default priority,
    // non-blocking) and their events
    hipStream_t side = nullptr, opt = nullptr;
    std::vector<hipEvent_t> evs;
    // scratch of the weight-gradient stream: split-K partials and column-sum
    // slices of every weight and bias gradient (they run there one at a time)
    Ws wscratch{nullptr, 0};
    int32_t *route_e = nullptr, *perm = nullptr, *off = nullptr, *emb_b = nullptr, *emb_perm = nullptr,
            *emb_off = nullptr;
    void *route_ws = nullptr, *emb_ws = nullptr;
    bool fwd_done = false;
    MDecode dec;
};

static void free_acts(asca_model* M) {
    if (!M->allocs.empty()) (void)hipDeviceSynchronize();
    for (void* a : M->allocs) (void)hipFree(a);
    M->allocs.clear();
    M->acts.clear();
    M->wscratch = Ws{nullptr, 0};
    M->batch = M->seq = 0;
    M->fwd_done = false;
}

template <typename T>
static int dalloc(asca_model* M, T** out, size_t count) {
    void* p = nullptr;
    const size_t bytes = (count ? count : 1) * sizeof(T);
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return fail(ASCA_ERR_OOM, "model: hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    M->allocs.push_back(p);
    *out = reinterpret_cast<T*>(p);
    return ASCA_OK;
}

static int ensure_acts(asca_model* M, int batch, int seq) {
    if (M->batch == batch && M->seq == seq) return ASCA_OK;
    free_acts(M);
    const size_t T = (size_t)batch * seq, d = M->d, H = M->H, dff = M->dff, V = M->V;
    size_t dws = 0;
    int rc = asca_delta_ws_bytes(batch, seq, M->H, M->dh, &dws);
    if (rc) return rc;
    size_t rws = 0, ews = 0;
    if ((rc = asca_hash_route_ws_bytes((int)T, M->E, &rws)) || (rc = asca_hash_route_ws_bytes((int)T, M->V, &ews)))
        return rc;
    M->acts.resize(M->L);
    for (int l = 0; l < M->L; ++l) {
        MActs& a = M->acts[l];
        char* dw = nullptr;
        if ((rc = dalloc(M, &a.x_out, T * d)) || (rc = dalloc(M, &a.q, T * d)) || (rc = dalloc(M, &a.k, T * d)) ||
            (rc = dalloc(M, &a.v, T * d)) || (rc = dalloc(M, &a.qn, T * H)) || (rc = dalloc(M, &a.kn, T * H)) ||
            (rc = dalloc(M, &a.al, T * H)) || (rc = dalloc(M, &a.be, T * H)) || (rc = dalloc(M, &a.o, T * d)) ||
            (rc = dalloc(M, &a.x_mid, T * d)) || (rc = dalloc(M, &a.xn, T * d)) ||
            (rc = dalloc(M, &a.pre, T * dff)) || (rc = dalloc(M, &a.hid, T * dff)) || (rc = dalloc(M, &dw, dws)))
            goto oom;
        a.dws = dw;
    }
    {
        char *rw = nullptr, *ew = nullptr;
        if ((rc = dalloc(M, &M->x0, T * d)) || (rc = dalloc(M, &M->qkv_t, T * 3 * d)) ||
            (rc = dalloc(M, &M->gate_t, T * 2 * H)) || (rc = dalloc(M, &M->h_final, T * d)) ||
            (rc = dalloc(M, &M->logits, T * V)) || (rc = dalloc(M, &M->dlogits, T * V)) ||
            (rc = dalloc(M, &M->losses, T)) || (rc = dalloc(M, &M->loss, 1)) || (rc = dalloc(M, &M->dxn, T * d)) ||
            (rc = dalloc(M, &M->dtmp, T * d)) ||
            (rc = dalloc(M, &M->route_e, T)) || (rc = dalloc(M, &M->perm, T)) ||
            (rc = dalloc(M, &M->off, (size_t)M->E + 1)) || (rc = dalloc(M, &M->emb_b, T)) ||
            (rc = dalloc(M, &M->emb_perm, T)) || (rc = dalloc(M, &M->emb_off, V + 1)) ||
            (rc = dalloc(M, &rw, rws)) || (rc = dalloc(M, &ew, ews)))
            goto oom;
        M->route_ws = rw;
        M->emb_ws = ew;
        // the weight-gradient stream's scratch, for its largest user
        size_t ws = gemm_ws_floats(d, V, (int)T);
        ws = std::max(ws, gemm_ws_floats(d, d, (int)T));
        ws = std::max(ws, gemm_ws_floats(d, 3 * d, (int)T));
        ws = std::max(ws, colsum_ws_floats((long)T, d, false, 0));
        ws = std::max(ws, colsum_ws_floats((long)T, 3 * d, false, 0));
        ws = std::max(ws, skinny_wgrad_ws_floats((long)T, d, 2 * H));
        ws = std::max(ws, moe_bwd_weights_ws_floats((int)T, d, dff, M->E));
        float* wsp = nullptr;
        if ((rc = dalloc(M, &wsp, ws))) goto oom;
        M->wscratch = Ws{wsp, ws};
        for (int k = 0; k < 2; ++k)
            if ((rc = dalloc(M, &M->dx[k], T * d)) || (rc = dalloc(M, &M->dmid[k], T * d)) ||
                (rc = dalloc(M, &M->dqkv[k], T * 3 * d)) || (rc = dalloc(M, &M->dgate[k], T * 2 * H)) ||
                (rc = dalloc(M, &M->dpre[k], T * dff)))
                goto oom;
    }
    M->batch = batch;
    M->seq = seq;
    return ASCA_OK;
oom:
    free_acts(M);
    return rc;
}

static GemmArgs gemm_plain(const float* A, long lda, const float* B, long ldb, float* C, long ldc, int M, int N, int K) {
    GemmArgs a = gemm_args();
    a.A = A;
    a.lda = lda;
    a.B = B;
    a.ldb = ldb;
    a.C = C;
    a.ldc = ldc;
    a.M = M;
    a.N = N;
    a.K = K;
    return a;
}

static int d2d(void* dst, const void* src, size_t bytes, hipStream_t st) {
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, st);
    return e == hipSuccess ? ASCA_OK : fail(ASCA_ERR_HIP, "hipMemcpyAsync: %s", hipGetErrorString(e));
}

// Forward of the whole model, keeping what the backward needs.
static int model_forward(asca_model* M, const uint32_t* ids, const uint32_t* targets, hipStream_t st) {
    const int T = M->batch * M->seq, d = M->d, H = M->H, dh = M->dh, E = M->E, dff = M->dff, V = M->V;
    int rc;
    // routing of this batch (the same ids for every layer) and the id buckets
    if ((rc = bucket_launch(true, ids, T, E, M->route_e, M->perm, M->off, M->route_ws, st))) return rc;
    if ((rc = bucket_launch(false, ids, T, V, M->emb_b, M->emb_perm, M->emb_off, M->emb_ws, st))) return rc;
    if ((rc = pre_launch("embed"))) return rc;
    hipLaunchKernelGGL(embed_k, dim3((T + 3) / 4), dim3(256), 0, st, M->p + M->t[0].off, ids, (long)T, d, V, M->x0);
    if ((rc = post_launch("embed"))) return rc;
    const float* x = M->x0;
    for (int l = 0; l < M->L; ++l) {
        const MLayer& P = M->lay[l];
        MActs& a = M->acts[l];
        // qkv = x W_qkv + b_qkv ; gate = x W_gate + b_gate
        GemmArgs q = gemm_plain(x, d, M->p + P.w_qkv, 3 * d, M->qkv_t, 3 * d, T, 3 * d, d);
        q.bias = M->p + P.b_qkv;
        if ((rc = gemm_launch(0, 0, EPI_STORE, q, T, st, "qkv_proj"))) return rc;
        if ((rc = skinny_fwd_launch(x, d, M->p + P.w_gate, M->p + P.b_gate, M->gate_t, T, d, 2 * H, st))) return rc;
        if ((rc = pre_launch("qkv_prep"))) return rc;
        hipLaunchKernelGGL(qkv_prep_k, dim3(T), dim3(256), 0, st, M->qkv_t, M->gate_t, H, dh, a.q, a.k, a.v, a.qn,
                           a.kn, a.al, a.be);
        if ((rc = post_launch("qkv_prep"))) return rc;
        if ((rc = asca_delta_fwd(a.q, a.k, a.v, a.al, a.be, a.o, a.dws, M->batch, M->seq, H, dh, st))) return rc;
        // x_mid = x + (o W_o + b_o)
        GemmArgs yo = gemm_plain(a.o, d, M->p + P.w_o, d, a.x_mid, d, T, d, d);
        yo.bias = M->p + P.b_o;
        yo.resid = x;
        yo.ld_resid = d;
        if ((rc = gemm_launch(0, 0, EPI_STORE, yo, T, st, "out_proj"))) return rc;
        // MoE on RMSNorm(x_mid); x_out = x_mid + moe
        if ((rc = asca_rmsnorm(a.x_mid, a.xn, nullptr, T, d, MODEL_EPS, st))) return rc;
        GemmArgs w1 = gemm_args();
        w1.A = a.xn;
        w1.lda = d;
        w1.a_rows = M->perm;
        w1.B = M->p + P.w1;
        w1.ldb = (long)E * dff;
        w1.b_gs = dff;
        w1.C = a.pre;
        w1.ldc = dff;
        w1.bias = M->p + P.b1;
        w1.bias_gs = dff;
        w1.aux_out = a.hid;
        w1.ld_aux = dff;
        w1.M = T;
        w1.N = dff;
        w1.K = d;
        w1.goff = M->off;
        w1.ngroups = E;
        w1.gmode = 1;
        if ((rc = gemm_launch(0, 0, EPI_SILU, w1, T, st, "moe_fwd_w1"))) return rc;
        GemmArgs w2 = gemm_args();
        w2.A = a.hid;
        w2.lda = dff;
        w2.B = M->p + P.w2;
        w2.ldb = d;
        w2.b_gs = (long)dff * d;
        w2.C = a.x_out;
        w2.ldc = d;
        w2.c_rows = M->perm;
        w2.bias = M->p + P.b2;
        w2.resid = a.x_mid;
        w2.ld_resid = d;
        w2.M = T;
        w2.N = d;
        w2.K = dff;
        w2.goff = M->off;
        w2.ngroups = E;
        w2.gmode = 1;
        if ((rc = gemm_launch(0, 0, EPI_STORE, w2, T, st, "moe_fwd_w2"))) return rc;
        x = a.x_out;
    }
    // head and loss
    if ((rc = asca_rmsnorm(x, M->h_final, nullptr, T, d, MODEL_EPS, st))) return rc;
    GemmArgs hd = gemm_plain(M->h_final, d, M->p + M->t[1].off, V, M->logits, V, T, V, d);
    if ((rc = gemm_launch(0, 0, EPI_STORE, hd, T, st, "head"))) return rc;
    if ((rc = asca_cross_entropy(M->logits, targets, T, V, M->dlogits, M->losses, st))) return rc;
    if ((rc = pre_launch("loss_mean"))) return rc;
    hipLaunchKernelGGL(loss_mean_k, dim3(1), dim3(256), 0, st, M->losses, (long)T, 1.0f / (float)T, M->loss);
    if ((rc = post_launch("loss_mean"))) return rc;
    M->fwd_done = true;
    return ASCA_OK;
}

static int gemm_wgrad(const float* X, int ldx, const float* D, int ldd, float* G, int M_, int N_, int T, Ws ws,
                      hipStream_t st) {
    // G (M_ x N_) = X^T D over T rows; split K when the output is small
    return gemm_run(1, 0, M_, N_, T, 1.0f, X, ldx, D, ldd, 0.0f, G, N_, nullptr, ws, st);
}

// Weight-gradient and optimiser streams and their events, created on first
// use.  Events per layer l: 5l + {0: dpre written, 1: d_mid written, 2: d_qkv
// written, 3: the layer's weight gradients done, 4: the chain done with the
// layer's weights}; then EV_FORK, EV_JOIN (weight-gradient stream done),
// EV_HEAD_CHAIN (the chain done with the head weights), EV_HEAD_GRAD (head
// weight gradient done), EV_EMB (embedding gradient done), EV_OPT (optimiser
// stream done).
enum { EV_FORK = 0, EV_JOIN, EV_HEAD_CHAIN, EV_HEAD_GRAD, EV_EMB, EV_OPT, EV_GLOBAL };

static void drop_side(asca_model* M) {
    for (hipEvent_t x : M->evs)
        if (x) (void)hipEventDestroy(x);
    M->evs.clear();
    if (M->side) (void)hipStreamDestroy(M->side);
    if (M->opt) (void)hipStreamDestroy(M->opt);
    M->side = M->opt = nullptr;
}

static int ensure_side(asca_model* M) {
    if (M->side) return ASCA_OK;
    hipError_t e = hipStreamCreateWithFlags(&M->side, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&M->opt, hipStreamNonBlocking);
    if (e != hipSuccess) {
        drop_side(M);
        return fail(ASCA_ERR_HIP, "hipStreamCreateWithFlags: %s", hipGetErrorString(e));
    }
    M->evs.assign((size_t)5 * M->L + EV_GLOBAL, nullptr);
    for (auto& ev : M->evs)
        if ((e = hipEventCreateWithFlags(&ev, hipEventDisableTiming)) != hipSuccess) {
            // leave no half-made set behind: the next call starts again
            drop_side(M);
            return fail(ASCA_ERR_HIP, "hipEventCreateWithFlags: %s", hipGetErrorString(e));
        }
    return ASCA_OK;
}

// `from` records event ev, `to` waits for it.
static int hand_over(hipStream_t from, hipStream_t to, hipEvent_t ev) {
    hipError_t e = hipEventRecord(ev, from);
    if (e == hipSuccess) e = hipStreamWaitEvent(to, ev, 0);
    return e == hipSuccess ? (int)ASCA_OK : fail(ASCA_ERR_HIP, "stream hand-over: %s", hipGetErrorString(e));
}

// After a failure: `st` still waits for whatever was queued on `from`, so no
// later work on `st` races it.  Keeps the failure's message.
static void join_after_error(hipStream_t from, hipStream_t st, hipEvent_t ev) {
    if (hipEventRecord(ev, from) == hipSuccess) (void)hipStreamWaitEvent(st, ev, 0);
}

// Backward of the whole model into the gradient buffer (overwritten).
//
// The chain of data gradients (dx through each layer) runs on the caller's
// stream `st`.  The weight and bias gradients, which nothing later in the
// backward reads, run on the model's second stream as soon as their inputs
// are written, so they overlap the next layer's chain (above all the
// VALU-bound recurrence backward, which leaves the matrix cores idle).  The
// gradients they read alternate between two buffer sets by layer parity;
// before the chain overwrites a set it waits for the weight gradients that
// read it (layer l + 2, and layer l + 1 for dx), and `st` joins the second
// stream at the end, so work queued on `st` afterwards sees every gradient.
// On a failure `st` still joins what was queued on the second stream.
static int adamw_range(asca_model* M, size_t j0, size_t j1, hipStream_t st);

static int backward_body(asca_model* M, hipStream_t st, hipStream_t sd) {
    const int T = M->batch * M->seq, d = M->d, H = M->H, dh = M->dh, E = M->E, dff = M->dff, V = M->V, L = M->L;
    auto ev = [&](int l, int k) { return M->evs[(size_t)5 * l + k]; };
    auto gev = [&](int k) { return M->evs[(size_t)5 * L + k]; };
    const Ws ws = M->wscratch;
    float* G = M->g;
    const float* x_last = M->acts[L - 1].x_out;
    int rc;
    // head: d_head = h^T dlogits (second stream) ; dh = dlogits W_head^T ; dx = rmsnorm_bwd(x_L, dh)
    if ((rc = gemm_wgrad(M->h_final, d, M->dlogits, V, G + M->t[1].off, d, V, T, ws, sd))) return rc;
    if (hipEventRecord(gev(EV_HEAD_GRAD), sd) != hipSuccess) return fail(ASCA_ERR_HIP, "hipEventRecord failed");
    GemmArgs dhh = gemm_plain(M->dlogits, V, M->p + M->t[1].off, V, M->dtmp, d, T, d, V);
    if ((rc = gemm_launch(0, 1, EPI_STORE, dhh, T, st, "head_dx"))) return rc;
    if (hipEventRecord(gev(EV_HEAD_CHAIN), st) != hipSuccess) return fail(ASCA_ERR_HIP, "hipEventRecord failed");
    if ((rc = rmsnorm_bwd_launch(x_last, M->dtmp, nullptr, M->dx[(L - 1) & 1], T, d, MODEL_EPS, st))) return rc;
    for (int l = L - 1; l >= 0; --l) {
        const MLayer& P = M->lay[l];
        MActs& a = M->acts[l];
        const float* x_in = l ? M->acts[l - 1].x_out : M->x0;
        const int b = l & 1;
        float *din = M->dx[b], *dout = M->dx[b ^ 1], *dmid = M->dmid[b], *dqkv = M->dqkv[b], *dgate = M->dgate[b],
              *dpre = M->dpre[b];
        // set b was last read by the weight gradients of layer l + 2
        if (l + 2 < L && hipStreamWaitEvent(st, ev(l + 2, 3), 0) != hipSuccess)
            return fail(ASCA_ERR_HIP, "hipStreamWaitEvent failed");
        // MoE backward from dout = din; d_mid = din + rmsnorm_bwd(x_mid, dxn)
        if ((rc = moe_bwd_data(M->p + P.w1, M->p + P.w2, a.pre, M->perm, M->off, din, T, d, dff, E, M->dxn, dpre,
                               st)))
            return rc;
        if ((rc = hand_over(st, sd, ev(l, 0)))) return rc;
        if ((rc = moe_bwd_weights(a.xn, a.hid, M->perm, M->off, din, dpre, T, d, dff, E, G + P.w1, G + P.b1,
                                  G + P.w2, G + P.b2, 0, ws, sd)))
            return rc;
        if ((rc = rmsnorm_bwd_launch(a.x_mid, M->dxn, din, dmid, T, d, MODEL_EPS, st))) return rc;
        if ((rc = hand_over(st, sd, ev(l, 1)))) return rc;
        if ((rc = gemm_wgrad(a.o, d, dmid, d, G + P.w_o, d, d, T, ws, sd))) return rc;
        if ((rc = colsum_launch(dmid, T, d, d, nullptr, 0, G + P.b_o, 0, ws, sd))) return rc;
        // delta block backward (delta.rs:615-674) from dy = d_mid
        GemmArgs dov = gemm_plain(dmid, d, M->p + P.w_o, d, M->dtmp, d, T, d, d);
        if ((rc = gemm_launch(0, 1, EPI_STORE, dov, T, st, "out_proj_dx"))) return rc;
        if ((rc = asca_delta_bwd_fused(a.q, a.k, a.v, a.al, a.be, a.qn, a.kn, M->dtmp, a.dws, dqkv, dgate, M->batch,
                                       M->seq, H, dh, st)))
            return rc;
        if ((rc = hand_over(st, sd, ev(l, 2)))) return rc;
        if ((rc = gemm_wgrad(x_in, d, dqkv, 3 * d, G + P.w_qkv, d, 3 * d, T, ws, sd))) return rc;
        if ((rc = colsum_launch(dqkv, T, 3 * d, 3 * d, nullptr, 0, G + P.b_qkv, 0, ws, sd))) return rc;
        if ((rc = skinny_wgrad_launch(x_in, d, dgate, G + P.w_gate, G + P.b_gate, T, d, 2 * H, ws, sd))) return rc;
        if (hipEventRecord(ev(l, 3), sd) != hipSuccess) return fail(ASCA_ERR_HIP, "hipEventRecord failed");
        // dout (the layer below's din) was last read by the weight gradients of layer l + 1
        if (l + 1 < L && hipStreamWaitEvent(st, ev(l + 1, 3), 0) != hipSuccess)
            return fail(ASCA_ERR_HIP, "hipStreamWaitEvent failed");
        // dx = d_mid + d_qkv W_qkv^T + d_gate W_gate^T
        GemmArgs dq = gemm_plain(dqkv, 3 * d, M->p + P.w_qkv, 3 * d, dout, d, T, d, 3 * d);
        dq.resid = dmid;
        dq.ld_resid = d;
        if ((rc = gemm_launch(0, 1, EPI_STORE, dq, T, st, "qkv_proj_dx"))) return rc;
        GemmArgs dg = gemm_plain(dgate, 2 * H, M->p + P.w_gate, 2 * H, dout, d, T, d, 2 * H);
        dg.beta = 1.0f;
        if ((rc = gemm_launch(0, 1, EPI_STORE, dg, T, st, "gate_proj_dx"))) return rc;
        // the chain is done with layer l's weights
        if (hipEventRecord(ev(l, 4), st) != hipSuccess) return fail(ASCA_ERR_HIP, "hipEventRecord failed");
    }
    // embedding gradient
    if ((rc = pre_launch("embed_grad"))) return rc;
    hipLaunchKernelGGL(embed_grad_k, dim3(V), dim3(256), 0, st, M->dx[1], M->emb_perm, M->emb_off, d,
                       G + M->t[0].off);
    if ((rc = post_launch("embed_grad"))) return rc;
    if (hipEventRecord(gev(EV_EMB), st) != hipSuccess) return fail(ASCA_ERR_HIP, "hipEventRecord failed");
    return ASCA_OK;
}

// The optimiser step of a training step on the model's third stream: each
// group of tensors (head, layers from the top, embedding) starts once its
// gradients are final and the chain no longer reads its weights, so the
// updates overlap the rest of the backward (the update is elementwise per
// tensor: the result equals one launch after the backward).  Issued only
// after every backward launch was queued without error.
static int optimiser_body(asca_model* M, hipStream_t st, hipStream_t sd, int* launched) {
    const int L = M->L;
    auto ev = [&](int l, int k) { return M->evs[(size_t)5 * l + k]; };
    auto gev = [&](int k) { return M->evs[(size_t)5 * L + k]; };
    const hipStream_t so = M->opt;
    (void)sd;
    (void)st;
    auto group = [&](hipEvent_t a, hipEvent_t b, size_t j0, size_t j1) -> int {
        if (hipStreamWaitEvent(so, a, 0) != hipSuccess || hipStreamWaitEvent(so, b, 0) != hipSuccess)
            return fail(ASCA_ERR_HIP, "hipStreamWaitEvent failed");
        int rc = adamw_range(M, j0, j1, so);
        if (!rc) ++*launched;
        return rc;
    };
    int rc = group(gev(EV_HEAD_GRAD), gev(EV_HEAD_CHAIN), 1, 2);   // head (tensor 1)
    for (int l = L - 1; l >= 0 && !rc; --l)                         // layer l: tensors 2 + 10 l .. 2 + 10 l + 9
        rc = group(ev(l, 3), ev(l, 4), 2 + 10 * (size_t)l, 12 + 10 * (size_t)l);
    if (!rc) rc = group(gev(EV_EMB), gev(EV_EMB), 0, 1);             // embedding (tensor 0)
    return rc;
}

// with_adamw: also apply AdamW (optimiser_body); the caller advances the step
// counter on success.  A failure there after some tensors were updated is
// reported as ASCA_ERR_PARTIAL_UPDATE; every other failure leaves the
// parameters and moments untouched.
static int model_backward(asca_model* M, hipStream_t st, bool with_adamw = false) {
    int rc = ensure_side(M);
    if (rc) return rc;
    const hipStream_t sd = M->side;
    auto gev = [&](int k) { return M->evs[(size_t)5 * M->L + k]; };
    if ((rc = hand_over(st, sd, gev(EV_FORK)))) return rc;
    if ((rc = backward_body(M, st, sd))) {
        join_after_error(sd, st, gev(EV_JOIN));
        return rc;
    }
    if (with_adamw) {
        int launched = 0;
        if ((rc = optimiser_body(M, st, sd, &launched))) {
            join_after_error(sd, st, gev(EV_JOIN));
            join_after_error(M->opt, st, gev(EV_OPT));
            if (launched) {
                const std::string why = asca_last_error();
                return fail(ASCA_ERR_PARTIAL_UPDATE, "optimiser step failed after %d of its launches (%s)", launched,
                            why.c_str());
            }
            return rc;
        }
        if ((rc = hand_over(M->opt, st, gev(EV_OPT)))) {
            join_after_error(sd, st, gev(EV_JOIN));
            return fail(ASCA_ERR_PARTIAL_UPDATE, "optimiser stream join failed");
        }
    }
    return hand_over(sd, st, gev(EV_JOIN));
}

// AdamW over tensors j0 .. j1-1 with the step counter base M->adam_step (the
// caller advances it once all tensors are updated).
static int adamw_range(asca_model* M, size_t j0, size_t j1, hipStream_t st) {
    const int c0 = M->chunk0[j0], c1 = M->chunk0[j1];
    if (c1 <= c0) return ASCA_OK;
    int rc = pre_launch("adamw_multi");
    if (rc) return rc;
    hipLaunchKernelGGL(adamw_multi_k, dim3(c1 - c0), dim3(256), 0, st, M->p, M->g, M->m, M->v, M->chunks + c0,
                       M->adam_step, M->lr, M->b1, M->b2, M->eps, M->wd);
    return post_launch("adamw_multi");
}

static int model_adamw(asca_model* M, hipStream_t st) {
    int rc = adamw_range(M, 0, M->t.size(), st);
    if (rc) return rc;
    M->adam_step += (uint32_t)M->t.size();
    return ASCA_OK;
}

static void free_decode(asca_model* M) {
    if (!M->dec.allocs.empty()) (void)hipDeviceSynchronize();
    for (void* a : M->dec.allocs) (void)hipFree(a);
    M->dec = MDecode();
}

// Decode workspace for n sequences (one row each).
static int ensure_decode(asca_model* M, int n) {
    MDecode& D = M->dec;
    if (D.n == n) return ASCA_OK;
    free_decode(M);
    size_t rws = 0;
    int rc = asca_hash_route_ws_bytes(n, M->E, &rws);
    if (rc) return rc;
    const size_t d = M->d, N = n;
    auto take = [&](auto** out, size_t count, size_t elem) {
        void* p = nullptr;
        const size_t bytes = (count ? count : 1) * elem;
        hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) return fail(ASCA_ERR_OOM, "decode: hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
        D.allocs.push_back(p);
        *out = reinterpret_cast<std::remove_pointer_t<decltype(out)>>(p);
        return (int)ASCA_OK;
    };
    if ((rc = take(&D.xa, N * d, 4)) || (rc = take(&D.xb, N * d, 4)) || (rc = take(&D.qkv, N * 3 * d, 4)) ||
        (rc = take(&D.gate, N * 2 * M->H, 4)) || (rc = take(&D.o, N * d, 4)) || (rc = take(&D.mid, N * d, 4)) ||
        (rc = take(&D.xn, N * d, 4)) || (rc = take(&D.pre, N * M->dff, 4)) || (rc = take(&D.hid, N * M->dff, 4)) ||
        (rc = take(&D.hf, N * d, 4)) || (rc = take(&D.route, N, 4)) || (rc = take(&D.perm, N, 4)) ||
        (rc = take(&D.off, (size_t)M->E + 1, 4)) || (rc = take(&D.rws, rws, 1))) {
        free_decode(M);
        return rc;
    }
    D.n = n;
    return ASCA_OK;
}

// Model::step for n sequences, one token each (model.rs:631-649): embedding,
// per layer x_mid = x + DeltaBlock::step(x) (delta.rs:341-411, the layer's
// states) and x = x_mid + HashMoe::step(x_mid) (model.rs:308-337: RMSNorm, the
// token's hashed expert, SiLU, shared b2), then RMSNorm and the head.  The same
// launches as the training forward at one row per sequence, with the delta
// recurrence replaced by the decode step on the carried states.
static int model_decode(asca_model* M, const uint32_t* ids, int n, float* states, float* logits, hipStream_t st) {
    MDecode& D = M->dec;
    const int d = M->d, H = M->H, dh = M->dh, E = M->E, dff = M->dff, V = M->V;
    const size_t sl = (size_t)n * H * dh * dh;  // one layer's states
    int rc;
    if ((rc = bucket_launch(true, ids, n, E, D.route, D.perm, D.off, D.rws, st))) return rc;
    if ((rc = pre_launch("embed"))) return rc;
    hipLaunchKernelGGL(embed_k, dim3((n + 3) / 4), dim3(256), 0, st, M->p + M->t[0].off, ids, (long)n, d, V, D.xa);
    if ((rc = post_launch("embed"))) return rc;
    float* x = D.xa;
    float* nx = D.xb;
    for (int l = 0; l < M->L; ++l) {
        const MLayer& P = M->lay[l];
        GemmArgs q = gemm_plain(x, d, M->p + P.w_qkv, 3 * d, D.qkv, 3 * d, n, 3 * d, d);
        q.bias = M->p + P.b_qkv;
        if ((rc = gemm_launch(0, 0, EPI_STORE, q, n, st, "dec_qkv_proj"))) return rc;
        if ((rc = skinny_fwd_launch(x, d, M->p + P.w_gate, M->p + P.b_gate, D.gate, n, d, 2 * H, st))) return rc;
        if ((rc = asca_delta_decode_step(states + l * sl, D.qkv, D.gate, D.o, n, H, dh, st))) return rc;
        GemmArgs yo = gemm_plain(D.o, d, M->p + P.w_o, d, D.mid, d, n, d, d);
        yo.bias = M->p + P.b_o;
        yo.resid = x;
        yo.ld_resid = d;
        if ((rc = gemm_launch(0, 0, EPI_STORE, yo, n, st, "dec_out_proj"))) return rc;
        if ((rc = asca_rmsnorm(D.mid, D.xn, nullptr, n, d, MODEL_EPS, st))) return rc;
        GemmArgs w1 = gemm_args();
        w1.A = D.xn;
        w1.lda = d;
        w1.a_rows = D.perm;
        w1.B = M->p + P.w1;
        w1.ldb = (long)E * dff;
        w1.b_gs = dff;
        w1.C = D.pre;
        w1.ldc = dff;
        w1.bias = M->p + P.b1;
        w1.bias_gs = dff;
        w1.aux_out = D.hid;
        w1.ld_aux = dff;
        w1.M = n;
        w1.N = dff;
        w1.K = d;
        w1.goff = D.off;
        w1.ngroups = E;
        w1.gmode = 1;
        if ((rc = gemm_launch(0, 0, EPI_SILU, w1, n, st, "dec_moe_w1"))) return rc;
        GemmArgs w2 = gemm_args();
        w2.A = D.hid;
        w2.lda = dff;
        w2.B = M->p + P.w2;
        w2.ldb = d;
        w2.b_gs = (long)dff * d;
        w2.C = nx;
        w2.ldc = d;
        w2.c_rows = D.perm;
        w2.bias = M->p + P.b2;
        w2.resid = D.mid;
        w2.ld_resid = d;
        w2.M = n;
        w2.N = d;
        w2.K = dff;
        w2.goff = D.off;
        w2.ngroups = E;
        w2.gmode = 1;
        if ((rc = gemm_launch(0, 0, EPI_STORE, w2, n, st, "dec_moe_w2"))) return rc;
        std::swap(x, nx);
    }
    if ((rc = asca_rmsnorm(x, D.hf, nullptr, n, d, MODEL_EPS, st))) return rc;
    GemmArgs hd = gemm_plain(D.hf, d, M->p + M->t[1].off, V, logits, V, n, V, d);
    return gemm_launch(0, 0, EPI_STORE, hd, n, st, "dec_head");
}

static void destroy_model(asca_model* M) {
    free_acts(M);
    free_decode(M);
    (void)hipDeviceSynchronize();
    drop_side(M);
    for (void* q : {(void*)M->p, (void*)M->g, (void*)M->m, (void*)M->v, (void*)M->chunks})
        if (q) (void)hipFree(q);
    delete M;
}

extern "C" {

int asca_model_create(int vocab, int d_model, int n_heads, int n_layers, int n_experts, int d_ff, asca_model** out) {
    if (!out) return fail(ASCA_ERR_INVALID, "null output pointer");
    *out = nullptr;
    if (vocab < 1 || vocab > 256 || d_model < 1 || n_heads < 1 || d_model % n_heads || n_layers < 1 ||
        n_experts < 1 || n_experts > 256 || d_ff < 1)
        return fail(ASCA_ERR_INVALID, "model: bad config V=%d d=%d H=%d L=%d E=%d d_ff=%d", vocab, d_model, n_heads,
                    n_layers, n_experts, d_ff);
    if (d_model / n_heads > 128) return fail(ASCA_ERR_UNSUPPORTED, "model: head dim %d > 128", d_model / n_heads);
    int rc = ensure_device();
    if (rc) return rc;
    asca_model* M = new asca_model();
    M->V = vocab;
    M->d = d_model;
    M->H = n_heads;
    M->dh = d_model / n_heads;
    M->L = n_layers;
    M->E = n_experts;
    M->dff = d_ff;
    auto add = [&](const char* name, int rows, int cols) {
        const size_t n = (size_t)rows * cols;
        M->t.push_back({name, M->n_params, n, rows, cols});
        M->n_params += (n + 3) / 4 * 4;  // 16-byte aligned tensor starts
        return M->t.back().off;
    };
    const int d = d_model, H = n_heads;
    add("embed", vocab, d);
    add("head", d, vocab);
    for (int l = 0; l < n_layers; ++l) {
        MLayer P;
        P.w_qkv = add("delta.w_qkv", d, 3 * d);
        P.b_qkv = add("delta.b_qkv", 1, 3 * d);
        P.w_gate = add("delta.w_gate", d, 2 * H);
        P.b_gate = add("delta.b_gate", 1, 2 * H);
        P.w_o = add("delta.w_o", d, d);
        P.b_o = add("delta.b_o", 1, d);
        P.w1 = add("moe.w1", d, n_experts * d_ff);
        P.b1 = add("moe.b1", 1, n_experts * d_ff);
        P.w2 = add("moe.w2", n_experts * d_ff, d);
        P.b2 = add("moe.b2", 1, d);
        M->lay.push_back(P);
    }
    // AdamW chunk table
    std::vector<AdamChunk> ch;
    const long CH = 16384;
    for (size_t j = 0; j < M->t.size(); ++j)
        for (long s = 0; s < (long)M->t[j].n; s += CH)
            ch.push_back({(int)j, 0, (long)M->t[j].off + s, std::min(CH, (long)M->t[j].n - s)});
    M->n_chunks = (int)ch.size();
    M->chunk0.assign(M->t.size() + 1, 0);
    for (size_t j = 0, c = 0; j <= M->t.size(); ++j) {
        while (c < ch.size() && (size_t)ch[c].tensor < j) ++c;
        M->chunk0[j] = (int)c;
    }
    const size_t bytes = M->n_params * sizeof(float);
    hipError_t e = hipSuccess;
    for (float** q : {&M->p, &M->g, &M->m, &M->v}) {
        if ((e = hipMalloc(q, bytes)) != hipSuccess) break;
        if ((e = hipMemset(*q, 0, bytes)) != hipSuccess) break;
    }
    if (e == hipSuccess) e = hipMalloc(&M->chunks, ch.size() * sizeof(AdamChunk));
    if (e == hipSuccess) e = hipMemcpy(M->chunks, ch.data(), ch.size() * sizeof(AdamChunk), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        destroy_model(M);
        return fail(ASCA_ERR_OOM, "model: allocation of %zu parameters failed: %s", M->n_params, hipGetErrorString(e));
    }
    *out = M;
    return ASCA_OK;
}

int asca_model_destroy(asca_model* M) {
    if (M) destroy_model(M);
    return ASCA_OK;
}

int asca_model_num_tensors(const asca_model* M, int* n) {
    if (!M || !n) return fail(ASCA_ERR_INVALID, "null pointer");
    *n = (int)M->t.size();
    return ASCA_OK;
}

int asca_model_tensor_info(const asca_model* M, int i, char* name, int name_len, size_t* offset, int* rows,
                           int* cols) {
    if (!M || i < 0 || i >= (int)M->t.size()) return fail(ASCA_ERR_INVALID, "tensor index %d out of range", i);
    const MTensor& t = M->t[i];
    if (name && name_len > 0) {
        snprintf(name, name_len, "%s", t.name.c_str());
    }
    if (offset) *offset = t.off;
    if (rows) *rows = t.rows;
    if (cols) *cols = t.cols;
    return ASCA_OK;
}

int asca_model_buffers(asca_model* M, size_t* n_floats, float** params, float** grads, float** m, float** v) {
    if (!M) return fail(ASCA_ERR_INVALID, "null model");
    if (n_floats) *n_floats = M->n_params;
    if (params) *params = M->p;
    if (grads) *grads = M->g;
    if (m) *m = M->m;
    if (v) *v = M->v;
    return ASCA_OK;
}

int asca_model_set_adamw(asca_model* M, float lr, float beta1, float beta2, float eps, float wd, uint32_t step) {
    if (!M) return fail(ASCA_ERR_INVALID, "null model");
    M->lr = lr;
    M->b1 = beta1;
    M->b2 = beta2;
    M->eps = eps;
    M->wd = wd;
    M->adam_step = step;
    return ASCA_OK;
}

int asca_model_adamw_step_count(const asca_model* M, uint32_t* step) {
    if (!M || !step) return fail(ASCA_ERR_INVALID, "null pointer");
    *step = M->adam_step;
    return ASCA_OK;
}

int asca_model_forward_backward(asca_model* M, const uint32_t* ids, const uint32_t* targets, int batch, int seq,
                                float* loss, void* stream) {
    if (!M || !ids || !targets) return fail(ASCA_ERR_INVALID, "null pointer");
    if (batch < 1 || seq < 1 || (long)batch * seq > 0x7fffffffL) return fail(ASCA_ERR_INVALID, "bad batch/seq");
    int rc = ensure_acts(M, batch, seq);
    if (rc) return rc;
    const hipStream_t st = as_stream(stream);
    if ((rc = model_forward(M, ids, targets, st))) return rc;
    if ((rc = model_backward(M, st))) return rc;
    if (loss) return d2d(loss, M->loss, sizeof(float), st);
    return ASCA_OK;
}

int asca_model_adamw(asca_model* M, void* stream) {
    if (!M) return fail(ASCA_ERR_INVALID, "null model");
    return model_adamw(M, as_stream(stream));
}

int asca_model_train_step(asca_model* M, const uint32_t* ids, const uint32_t* targets, int batch, int seq,
                          float* loss, void* stream) {
    if (!M || !ids || !targets) return fail(ASCA_ERR_INVALID, "null pointer");
    if (batch < 1 || seq < 1 || (long)batch * seq > 0x7fffffffL) return fail(ASCA_ERR_INVALID, "bad batch/seq");
    int rc = ensure_acts(M, batch, seq);
    if (rc) return rc;
    const hipStream_t st = as_stream(stream);
    if ((rc = model_forward(M, ids, targets, st))) return rc;
    if ((rc = model_backward(M, st, true))) return rc;
    M->adam_step += (uint32_t)M->t.size();
    if (loss) return d2d(loss, M->loss, sizeof(float), st);
    return ASCA_OK;
}

int asca_model_decode_state_floats(const asca_model* M, size_t* per_seq) {
    if (!M || !per_seq) return fail(ASCA_ERR_INVALID, "null pointer");
    *per_seq = (size_t)M->L * M->H * M->dh * M->dh;
    return ASCA_OK;
}

int asca_model_decode_step(asca_model* M, const uint32_t* ids, int n_seq, float* states, float* logits,
                           void* stream) {
    if (!M || !ids || !states || !logits) return fail(ASCA_ERR_INVALID, "null pointer");
    if (n_seq < 1 || (long)n_seq * M->H > 0x7fffffffL) return fail(ASCA_ERR_INVALID, "bad n_seq %d", n_seq);
    int rc = ensure_decode(M, n_seq);
    if (rc) return rc;
    return model_decode(M, ids, n_seq, states, logits, as_stream(stream));
}

}  // extern "C"
