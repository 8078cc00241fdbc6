/*
 * oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU f32 restatement of the reference crate's CPU path for the gated
 * delta-rule hot path (MythEclipse/asca, rust/src).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker / the timed CPU baseline.  Nothing in
 * the product (asca_amd/) links, loads or calls it.
 *
 * Every function cites the reference file:line it restates.  Rounding
 * follows the reference where that is cheap to mirror:
 *   - plain Rust loops never contract a*b+c into an FMA, so this file is
 *     compiled with -ffp-contract=off and writes those loops as mul + add;
 *   - simd::dot / simd::axpy / simd::scale_axpy (rust/src/simd.rs:27-206)
 *     use AVX2 8-lane FMA bodies with the same horizontal-sum order and a
 *     scalar tail, selected at run time exactly as simd::has_avx2 does;
 *   - the threading mirrors scan_cpu (one thread per head, delta.rs:262-321)
 *     and bptt_cpu (one thread per (head, sequence), delta.rs:446-575) so the
 *     timed baseline has the reference's decomposition.
 *
 * Parity pins (tests/test_oracle.py): golden vectors under tests/golden/,
 * the closed forms of the delta rule, finite differences, a float64 torch
 * autograd restatement written from the equations, and the batch/sequence
 * isolation and decode==forward invariants of the reference's own tests.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>

#define ORC_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------ simd */
/* rust/src/simd.rs:14-25: AVX2+FMA detected once at run time. */
static int g_avx2 = -1;
static int has_avx2(void) {
    if (g_avx2 < 0) {
        const char* e = getenv("ASCA_NO_SIMD");
        if (e && strcmp(e, "1") == 0) g_avx2 = 0;
        else g_avx2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    }
    return g_avx2;
}

__attribute__((target("avx2,fma")))
static float dot_avx2(const float* a, const float* b, int n) {
    /* rust/src/simd.rs:156-182 */
    int i = 0;
    __m256 acc = _mm256_setzero_ps();
    for (; i + 8 <= n; i += 8)
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc);
    __m128 hi = _mm256_extractf128_ps(acc, 1);
    __m128 lo = _mm256_castps256_ps128(acc);
    __m128 s = _mm_add_ps(hi, lo);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    float total = _mm_cvtss_f32(s);
    for (; i < n; ++i) total += a[i] * b[i];
    return total;
}

__attribute__((target("avx2,fma")))
static void axpy_avx2(float* dst, float a, const float* src, int n) {
    /* rust/src/simd.rs:136-154 */
    int i = 0;
    __m256 av = _mm256_set1_ps(a);
    for (; i + 8 <= n; i += 8)
        _mm256_storeu_ps(dst + i, _mm256_fmadd_ps(av, _mm256_loadu_ps(src + i), _mm256_loadu_ps(dst + i)));
    for (; i < n; ++i) dst[i] += a * src[i];
}

__attribute__((target("avx2,fma")))
static void scale_axpy_avx2(float* dst, float a, float b, const float* src, int n) {
    /* rust/src/simd.rs:114-134: dst = fma(b, src, a*dst) */
    int i = 0;
    __m256 av = _mm256_set1_ps(a), bv = _mm256_set1_ps(b);
    for (; i + 8 <= n; i += 8) {
        __m256 d = _mm256_loadu_ps(dst + i);
        __m256 s = _mm256_loadu_ps(src + i);
        _mm256_storeu_ps(dst + i, _mm256_fmadd_ps(bv, s, _mm256_mul_ps(av, d)));
    }
    for (; i < n; ++i) dst[i] = a * dst[i] + b * src[i];
}

/* rust/src/simd.rs:40-53 */
static float sdot(const float* a, const float* b, int n) {
    if (has_avx2()) return dot_avx2(a, b, n);
    float acc = 0.0f;
    for (int i = 0; i < n; ++i) acc += a[i] * b[i];
    return acc;
}
/* rust/src/simd.rs:27-38 */
static void saxpy(float* dst, float a, const float* src, int n) {
    if (has_avx2()) { axpy_avx2(dst, a, src, n); return; }
    for (int i = 0; i < n; ++i) dst[i] += a * src[i];
}
/* rust/src/simd.rs:70-80 (the AVX2 body is a plain per-lane multiply) */
static void sscale(float* dst, float a, int n) {
    for (int i = 0; i < n; ++i) dst[i] *= a;
}
/* rust/src/simd.rs:82-93 */
static void sscale_axpy(float* dst, float a, float b, const float* src, int n) {
    if (has_avx2()) { scale_axpy_avx2(dst, a, b, src, n); return; }
    for (int i = 0; i < n; ++i) dst[i] = a * dst[i] + b * src[i];
}

ORC_API int orc_has_avx2(void) { return has_avx2(); }
ORC_API float orc_sdot(const float* a, const float* b, int n) { return sdot(a, b, n); }

/* ------------------------------------------------------------------- rng */
/* rust/src/tensor.rs:299-337 (xorshift128+, Box-Muller in f32). */
typedef struct { uint64_t s0, s1; } orc_rng;

static void rng_init(orc_rng* r, uint64_t seed) {
    r->s0 = (seed * 0x9E3779B97F4A7C15ULL) | 1ULL;
    r->s1 = ((seed ^ 0xDEADBEEFCAFEF00DULL) * 0xBF58476D1CE4E5B9ULL) | 1ULL;
}
static uint64_t rng_next(orc_rng* r) {
    uint64_t x = r->s0;
    uint64_t y = r->s1;
    r->s0 = y;
    x ^= x << 23;
    r->s1 = x ^ y ^ (x >> 17) ^ (y >> 26);
    return r->s1 + y;
}
static float rng_uniform(orc_rng* r) {
    return (float)(rng_next(r) >> 40) / (float)(1u << 24);
}
static float rng_normal(orc_rng* r) {
    float u1 = rng_uniform(r);
    if (!(u1 >= 1e-7f)) u1 = 1e-7f; /* f32::max(u1, 1e-7) */
    float u2 = rng_uniform(r);
    const float two_pi = 2.0f * 3.14159265358979323846f;
    return sqrtf(-2.0f * logf(u1)) * cosf(two_pi * u2);
}

ORC_API void orc_rng_u64(uint64_t seed, uint64_t* out, int n) {
    orc_rng r; rng_init(&r, seed);
    for (int i = 0; i < n; ++i) out[i] = rng_next(&r);
}
ORC_API void orc_rng_normal(uint64_t seed, float* out, long n) {
    orc_rng r; rng_init(&r, seed);
    for (long i = 0; i < n; ++i) out[i] = rng_normal(&r);
}

/* rust/src/tensor.rs:245-248 */
static float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

/* ------------------------------------------------------- delta: L2 norm */
/* rust/src/delta.rs:145-165: per (row, head) x/max(||x||, 1e-8), norm saved. */
ORC_API void orc_l2norm_heads(float* x, float* norms, long rows, int H, int dh) {
    for (long r = 0; r < rows; ++r)
        for (int h = 0; h < H; ++h) {
            float* seg = x + r * (long)H * dh + (long)h * dh;
            float s = 0.0f;
            for (int c = 0; c < dh; ++c) s += seg[c] * seg[c];
            float n = sqrtf(s);
            if (!(n >= 1e-8f)) n = 1e-8f;
            for (int c = 0; c < dh; ++c) seg[c] /= n;
            if (norms) norms[r * H + h] = n;
        }
}

/* Synthetic inputs of the benchmark configs, in the fixed order
 * q, k, v (normal), alpha logits 2+normal, beta logits normal, dO (normal);
 * then q, k are L2-normalised per head and alpha, beta = sigmoid(logits). */
ORC_API void orc_delta_inputs(uint64_t seed, int B, int T, int H, int dh,
                              float* q, float* k, float* v, float* alpha, float* beta,
                              float* d_o, float* qn, float* kn, float* gate_logits) {
    orc_rng r; rng_init(&r, seed);
    long n = (long)B * T * H * dh, ng = (long)B * T * H;
    for (long i = 0; i < n; ++i) q[i] = rng_normal(&r);
    for (long i = 0; i < n; ++i) k[i] = rng_normal(&r);
    for (long i = 0; i < n; ++i) v[i] = rng_normal(&r);
    for (long i = 0; i < ng; ++i) alpha[i] = 2.0f + rng_normal(&r);
    for (long i = 0; i < ng; ++i) beta[i] = rng_normal(&r);
    if (d_o) for (long i = 0; i < n; ++i) d_o[i] = rng_normal(&r);
    orc_l2norm_heads(q, qn, (long)B * T, H, dh);
    orc_l2norm_heads(k, kn, (long)B * T, H, dh);
    for (long rr = 0; rr < (long)B * T; ++rr)
        for (int h = 0; h < H; ++h) {
            long i = rr * H + h;
            if (gate_logits) {
                gate_logits[rr * 2 * H + h] = alpha[i];
                gate_logits[rr * 2 * H + H + h] = beta[i];
            }
            alpha[i] = sigmoidf_(alpha[i]);
            beta[i] = sigmoidf_(beta[i]);
        }
}

/* ----------------------------------------------------- delta: forward scan */
/* One (head, sequence) unit of DeltaBlock::scan_cpu, rust/src/delta.rs:275-317.
 * states (nullable) receives (T+1)*dh*dh floats: S before every step, then
 * the final state. */
static void scan_unit(const float* q, const float* k, const float* v,
                      const float* alpha, const float* beta, int b, int h,
                      int T, int H, int dh, float* o, float* states,
                      float* s, float* sk, float* u) {
    const long d = (long)H * dh;
    const int off = h * dh;
    memset(s, 0, sizeof(float) * dh * dh);
    for (int t = 0; t < T; ++t) {
        long r = (long)b * T + t;
        if (states) memcpy(states + (long)t * dh * dh, s, sizeof(float) * dh * dh);
        const float* kt = k + r * d + off;
        const float* vt = v + r * d + off;
        float a = alpha[r * H + h];
        float bb = beta[r * H + h];
        for (int i = 0; i < dh; ++i) sk[i] = 0.0f;
        for (int ai = 0; ai < dh; ++ai) {               /* delta.rs:289-298 */
            float ka = kt[ai];
            if (ka == 0.0f) continue;
            const float* srow = s + (long)ai * dh;
            for (int i = 0; i < dh; ++i) sk[i] += srow[i] * ka;
        }
        for (int i = 0; i < dh; ++i) u[i] = bb * (vt[i] - a * sk[i]);   /* :299-301 */
        for (int ai = 0; ai < dh; ++ai)                                  /* :302-306 */
            for (int i = 0; i < dh; ++i)
                s[ai * dh + i] = a * s[ai * dh + i] + kt[ai] * u[i];
        const float* qt = q + r * d + off;                               /* :307-314 */
        for (int i = 0; i < dh; ++i) {
            float acc = 0.0f;
            for (int ai = 0; ai < dh; ++ai) acc += s[ai * dh + i] * qt[ai];
            o[r * d + off + i] = acc;
        }
    }
    if (states) memcpy(states + (long)T * dh * dh, s, sizeof(float) * dh * dh);
}

typedef struct {
    const float *q, *k, *v, *alpha, *beta;
    float *o, *states;
    int B, T, H, dh, h;
} scan_job;

static void* scan_head_thread(void* p) {
    /* delta.rs:274-319: one thread per head loops over the batch */
    scan_job* j = (scan_job*)p;
    float* s = malloc(sizeof(float) * j->dh * j->dh);
    float* sk = malloc(sizeof(float) * j->dh);
    float* u = malloc(sizeof(float) * j->dh);
    for (int b = 0; b < j->B; ++b) {
        float* st = j->states ? j->states + ((long)j->h * j->B + b) * (long)(j->T + 1) * j->dh * j->dh : NULL;
        scan_unit(j->q, j->k, j->v, j->alpha, j->beta, b, j->h, j->T, j->H, j->dh, j->o, st, s, sk, u);
    }
    free(s); free(sk); free(u);
    return NULL;
}

/* DeltaBlock::scan_cpu, rust/src/delta.rs:244-334.  states layout is the
 * reference's s_pre: unit (h*B + b), (T+1)*dh*dh floats each. */
ORC_API void orc_delta_scan(const float* q, const float* k, const float* v,
                            const float* alpha, const float* beta,
                            int B, int T, int H, int dh, float* o, float* states) {
    pthread_t* th = malloc(sizeof(pthread_t) * H);
    scan_job* jobs = malloc(sizeof(scan_job) * H);
    for (int h = 0; h < H; ++h) {
        jobs[h] = (scan_job){q, k, v, alpha, beta, o, states, B, T, H, dh, h};
        pthread_create(&th[h], NULL, scan_head_thread, &jobs[h]);
    }
    for (int h = 0; h < H; ++h) pthread_join(th[h], NULL);
    free(th); free(jobs);
}

/* --------------------------------------------------------- delta: BPTT */
/* One (head, sequence) job of DeltaBlock::bptt_cpu, rust/src/delta.rs:475-572.
 * Writes the raw per-head gradients (before the L2-norm and sigmoid
 * backward) straight into the (B*T, H*dh) / (B*T, H) outputs. */
static void bptt_unit(const float* q, const float* k, const float* v,
                      const float* alpha, const float* beta, const float* d_o,
                      const float* states, int b, int h, int T, int H, int dh,
                      float* dq_out, float* dk_out, float* dv_out,
                      float* da_out, float* db_out) {
    const long d = (long)H * dh;
    const int off = h * dh;
    float* ds = calloc((size_t)dh * dh, sizeof(float));
    float* ds_prev = calloc((size_t)dh * dh, sizeof(float));
    float* sk = calloc(dh, sizeof(float));
    float* u = calloc(dh, sizeof(float));
    float* dq = calloc(dh, sizeof(float));
    float* dk = calloc(dh, sizeof(float));
    float* du = calloc(dh, sizeof(float));
    float* dsk = calloc(dh, sizeof(float));
    for (int t = T - 1; t >= 0; --t) {
        for (int i = 0; i < dh; ++i) dk[i] = 0.0f;                 /* :489 */
        long r = (long)b * T + t;
        const float* s_t = states + (long)(t + 1) * dh * dh;
        const float* s_prev = states + (long)t * dh * dh;
        const float* qt = q + r * d + off;
        const float* kt = k + r * d + off;
        const float* vt = v + r * d + off;
        float a = alpha[r * H + h];
        float bb = beta[r * H + h];
        const float* do_t = d_o + r * d + off;
        for (int ai = 0; ai < dh; ++ai) dq[ai] = sdot(do_t, s_t + (long)ai * dh, dh);   /* :504-507 */
        for (int ai = 0; ai < dh; ++ai) {                                               /* :508-511 */
            dq_out[r * d + off + ai] = 0.0f + dq[ai];
            saxpy(ds + (long)ai * dh, qt[ai], do_t, dh);
        }
        for (int i = 0; i < dh; ++i) sk[i] = 0.0f;                                      /* :514-524 */
        for (int ai = 0; ai < dh; ++ai) {
            float ka = kt[ai];
            if (ka != 0.0f) saxpy(sk, ka, s_prev + (long)ai * dh, dh);
        }
        for (int i = 0; i < dh; ++i) u[i] = bb * (vt[i] - a * sk[i]);                   /* :525-527 */
        float dalpha = sdot(ds, s_prev, dh * dh);                                       /* :530 */
        float dbeta = 0.0f;
        for (int ai = 0; ai < dh; ++ai) dk[ai] += sdot(ds + (long)ai * dh, u, dh);      /* :532-534 */
        for (int i = 0; i < dh; ++i) du[i] = 0.0f;                                      /* :536-542 */
        for (int ai = 0; ai < dh; ++ai) {
            float ka = kt[ai];
            if (ka != 0.0f) saxpy(du, ka, ds + (long)ai * dh, dh);
        }
        for (long idx = 0; idx < (long)dh * dh; ++idx) ds_prev[idx] = a * ds[idx];     /* :543-545 */
        for (int i = 0; i < dh; ++i) {                                                  /* :548-553 */
            dbeta += du[i] * (vt[i] - a * sk[i]);
            dv_out[r * d + off + i] = 0.0f + bb * du[i];
            dsk[i] = -bb * a * du[i];
            dalpha += -bb * du[i] * sk[i];
        }
        for (int ai = 0; ai < dh; ++ai) {                                               /* :556-564 */
            const float* srow = s_prev + (long)ai * dh;
            dk[ai] += sdot(srow, dsk, dh);
            saxpy(ds_prev + (long)ai * dh, kt[ai], dsk, dh);
        }
        for (int ai = 0; ai < dh; ++ai) dk_out[r * d + off + ai] = 0.0f + dk[ai];       /* :566-568 */
        da_out[r * H + h] = dalpha;                                                      /* :569-570 */
        db_out[r * H + h] = dbeta;
        memcpy(ds, ds_prev, sizeof(float) * dh * dh);                                    /* :571 */
    }
    free(ds); free(ds_prev); free(sk); free(u); free(dq); free(dk); free(du); free(dsk);
}

typedef struct {
    const float *q, *k, *v, *alpha, *beta, *d_o, *states;
    float *dq, *dk, *dv, *da, *db;
    int B, T, H, dh, b, h;
} bptt_job;

static void* bptt_thread(void* p) {
    bptt_job* j = (bptt_job*)p;
    const float* st = j->states + ((long)j->h * j->B + j->b) * (long)(j->T + 1) * j->dh * j->dh;
    bptt_unit(j->q, j->k, j->v, j->alpha, j->beta, j->d_o, st, j->b, j->h, j->T, j->H, j->dh,
              j->dq, j->dk, j->dv, j->da, j->db);
    return NULL;
}

/* DeltaBlock::bptt_cpu raw part, rust/src/delta.rs:421-587: one thread per
 * (head, sequence), all spawned at once as std::thread::scope does. */
ORC_API void orc_delta_bptt_raw(const float* q, const float* k, const float* v,
                                const float* alpha, const float* beta, const float* d_o,
                                const float* states, int B, int T, int H, int dh,
                                float* dq, float* dk, float* dv, float* dalpha, float* dbeta) {
    int n = H * B;
    pthread_t* th = malloc(sizeof(pthread_t) * n);
    bptt_job* jobs = malloc(sizeof(bptt_job) * n);
    for (int h = 0; h < H; ++h)
        for (int b = 0; b < B; ++b) {
            int j = h * B + b;
            jobs[j] = (bptt_job){q, k, v, alpha, beta, d_o, states, dq, dk, dv, dalpha, dbeta, B, T, H, dh, b, h};
            pthread_create(&th[j], NULL, bptt_thread, &jobs[j]);
        }
    for (int j = 0; j < n; ++j) pthread_join(th[j], NULL);
    free(th); free(jobs);
}

/* norm_backward, rust/src/delta.rs:677-698: d = (d - y (y.d)) / s per head. */
ORC_API void orc_norm_backward(const float* y, const float* norms, float* dgrad,
                               long rows, int H, int dh) {
    for (long t = 0; t < rows; ++t)
        for (int h = 0; h < H; ++h) {
            long off = t * (long)H * dh + (long)h * dh;
            float s = norms[t * H + h];
            float dot = 0.0f;
            for (int c = 0; c < dh; ++c) dot += y[off + c] * dgrad[off + c];
            for (int c = 0; c < dh; ++c) dgrad[off + c] = (dgrad[off + c] - y[off + c] * dot) / s;
        }
}

/* The tail of bptt_cpu, rust/src/delta.rs:589-612: L2-norm backward of q, k,
 * concatenation into d_qkv (rows, 3d) and sigmoid backward into d_gate
 * (rows, 2H).  dq, dk are modified in place. */
ORC_API void orc_delta_fuse_grads(const float* q, const float* k, const float* qn, const float* kn,
                                  const float* alpha, const float* beta,
                                  float* dq, float* dk, const float* dv,
                                  const float* dalpha, const float* dbeta,
                                  long rows, int H, int dh, float* d_qkv, float* d_gate) {
    long d = (long)H * dh;
    orc_norm_backward(q, qn, dq, rows, H, dh);
    orc_norm_backward(k, kn, dk, rows, H, dh);
    for (long r = 0; r < rows; ++r) {
        for (long c = 0; c < d; ++c) {
            d_qkv[r * 3 * d + c] = dq[r * d + c];
            d_qkv[r * 3 * d + d + c] = dk[r * d + c];
            d_qkv[r * 3 * d + 2 * d + c] = dv[r * d + c];
        }
        for (int h = 0; h < H; ++h) {
            float al = alpha[r * H + h], be = beta[r * H + h];
            d_gate[r * 2 * H + h] = dalpha[r * H + h] * al * (1.0f - al);
            d_gate[r * 2 * H + H + h] = dbeta[r * H + h] * be * (1.0f - be);
        }
    }
}

/* ------------------------------------------- unit-wise fwd+BPTT (parity) */
/* Same per-unit arithmetic as orc_delta_scan + orc_delta_bptt_raw, but each
 * worker keeps only its own unit's (T+1)*dh*dh history, so configs whose
 * full history would not fit in memory can still be checked.  Outputs are
 * bit-identical to the reference-threaded drivers. */
typedef struct {
    const float *q, *k, *v, *alpha, *beta, *d_o;
    float *o, *dq, *dk, *dv, *da, *db;
    int B, T, H, dh;
    int next;          /* shared work counter (guarded by mu) */
    pthread_mutex_t mu;
} unit_pool;

static void* unit_worker(void* p) {
    unit_pool* P = (unit_pool*)p;
    int dh = P->dh;
    float* hist = malloc(sizeof(float) * (size_t)(P->T + 1) * dh * dh);
    float* s = malloc(sizeof(float) * dh * dh);
    float* sk = malloc(sizeof(float) * dh);
    float* u = malloc(sizeof(float) * dh);
    for (;;) {
        pthread_mutex_lock(&P->mu);
        int j = P->next++;
        pthread_mutex_unlock(&P->mu);
        if (j >= P->B * P->H) break;
        int h = j / P->B, b = j % P->B;
        scan_unit(P->q, P->k, P->v, P->alpha, P->beta, b, h, P->T, P->H, dh, P->o, hist, s, sk, u);
        if (P->d_o)
            bptt_unit(P->q, P->k, P->v, P->alpha, P->beta, P->d_o, hist, b, h, P->T, P->H, dh,
                      P->dq, P->dk, P->dv, P->da, P->db);
    }
    free(hist); free(s); free(sk); free(u);
    return NULL;
}

ORC_API void orc_delta_fwd_bwd_unitwise(const float* q, const float* k, const float* v,
                                        const float* alpha, const float* beta, const float* d_o,
                                        int B, int T, int H, int dh, int nthreads,
                                        float* o, float* dq, float* dk, float* dv,
                                        float* dalpha, float* dbeta) {
    unit_pool P = {q, k, v, alpha, beta, d_o, o, dq, dk, dv, dalpha, dbeta, B, T, H, dh, 0};
    pthread_mutex_init(&P.mu, NULL);
    if (nthreads < 1) nthreads = 1;
    pthread_t* th = malloc(sizeof(pthread_t) * nthreads);
    for (int i = 0; i < nthreads; ++i) pthread_create(&th[i], NULL, unit_worker, &P);
    for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
    pthread_mutex_destroy(&P.mu);
    free(th);
}

/* ------------------------------------------------------ delta: decode step */
/* State math of DeltaBlock::step, rust/src/delta.rs:356-407, for n_seq
 * independent sequences (the reference's fixed [0f32; 64] buffers at :361-362
 * are replaced by dh-sized ones, so dh > 64 works).  qkv: (n_seq, 3d) row as
 * produced by x.w_qkv + b_qkv; gate: (n_seq, 2H) logits; states:
 * (n_seq, H, dh, dh) updated in place; o: (n_seq, d). */
ORC_API void orc_delta_decode_step(float* states, const float* qkv, const float* gate,
                                   float* o, int n_seq, int H, int dh) {
    long d = (long)H * dh;
    float* qn = malloc(sizeof(float) * dh);
    float* kn = malloc(sizeof(float) * dh);
    float* sk = malloc(sizeof(float) * dh);
    float* u = malloc(sizeof(float) * dh);
    for (int n = 0; n < n_seq; ++n) {
        const float* row = qkv + (long)n * 3 * d;
        const float* grow = gate + (long)n * 2 * H;
        for (int hh = 0; hh < H; ++hh) {
            long off = (long)hh * dh;
            float a = sigmoidf_(grow[hh]);
            float b = sigmoidf_(grow[H + hh]);
            float qq = 0.0f, kk = 0.0f;
            for (int i = 0; i < dh; ++i) {
                float qv = row[off + i], kv = row[d + off + i];
                qq += qv * qv;
                kk += kv * kv;
            }
            float qs = sqrtf(qq); if (!(qs >= 1e-8f)) qs = 1e-8f;
            float ks = sqrtf(kk); if (!(ks >= 1e-8f)) ks = 1e-8f;
            float qi = 1.0f / qs, ki = 1.0f / ks;
            for (int i = 0; i < dh; ++i) {
                qn[i] = row[off + i] * qi;
                kn[i] = row[d + off + i] * ki;
            }
            float* s = states + ((long)n * H + hh) * dh * dh;
            for (int i = 0; i < dh; ++i) sk[i] = 0.0f;
            for (int ai = 0; ai < dh; ++ai) {
                float ka = kn[ai];
                if (ka == 0.0f) continue;
                saxpy(sk, ka, s + (long)ai * dh, dh);
            }
            for (int i = 0; i < dh; ++i) u[i] = b * (row[2 * d + off + i] - a * sk[i]);
            for (int ai = 0; ai < dh; ++ai) {
                float ka = kn[ai];
                if (ka == 0.0f) { sscale(s + (long)ai * dh, a, dh); continue; }
                sscale_axpy(s + (long)ai * dh, a, ka, u, dh);
            }
            for (int i = 0; i < dh; ++i) {
                float acc = 0.0f;
                for (int ai = 0; ai < dh; ++ai) acc += s[ai * dh + i] * qn[ai];
                o[(long)n * d + off + i] = acc;
            }
        }
    }
    free(qn); free(kn); free(sk); free(u);
}

/* -------------------------------------------------------------- RMSNorm */
/* rmsnorm_rows, rust/src/tensor.rs:259-270 (no gain). */
ORC_API void orc_rmsnorm(const float* x, float* y, long rows, int cols, float eps) {
    for (long r = 0; r < rows; ++r) {
        const float* row = x + r * cols;
        float ms = sdot(row, row, cols) / (float)cols;
        float inv = 1.0f / sqrtf(ms + eps);
        for (int c = 0; c < cols; ++c) y[r * cols + c] = row[c] * inv;
    }
}
/* rmsnorm_rows_backward, rust/src/tensor.rs:282-296. */
ORC_API void orc_rmsnorm_bwd(const float* x, const float* dy, float* dx, long rows, int cols, float eps) {
    for (long r = 0; r < rows; ++r) {
        const float* row = x + r * cols;
        const float* dyr = dy + r * cols;
        float ms = sdot(row, row, cols) / (float)cols;
        float inv = 1.0f / sqrtf(ms + eps);
        float mean = sdot(dyr, row, cols) * inv;
        mean /= (float)cols;
        for (int c = 0; c < cols; ++c) dx[r * cols + c] = inv * (dyr[c] - row[c] * inv * mean);
    }
}

/* ----------------------------------------------------------- hash route */
/* hash_route, rust/src/model.rs:69-77 (wrapping u32 arithmetic). */
ORC_API void orc_hash_route(const uint32_t* ids, long n, int n_experts, int32_t* out) {
    for (long i = 0; i < n; ++i) {
        uint32_t h = ids[i] * 0x9E3779B1u;
        h ^= h >> 15;
        h *= 0x85EBCA6Bu;
        h ^= h >> 13;
        out[i] = (int32_t)(h % (uint32_t)n_experts);
    }
}

/* ----------------------------------------------------------------- AdamW */
/* f32::powi(x, n) with a run-time exponent lowers to compiler-rt's
 * __powisf2: binary exponentiation by repeated squaring. */
static float powi_f32(float a, int b) {
    int recip = b < 0;
    float r = 1.0f;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

/* AdamW::update CPU body, rust/src/tensor.rs:392-402 and :444-453.  *step is
 * incremented once per call (once per parameter tensor, as the reference does). */
ORC_API void orc_adamw(float* p, const float* g, float* m, float* v, long n,
                       float lr, float beta1, float beta2, float eps, float wd, uint32_t* step) {
    *step += 1;
    float bc1 = 1.0f - powi_f32(beta1, (int)*step);
    float bc2 = 1.0f - powi_f32(beta2, (int)*step);
    float lrb = lr * sqrtf(bc1 / bc2);
    float eps_t = eps * sqrtf(bc2);
    float wdd = lr * wd;
    for (long i = 0; i < n; ++i) {
        float gi = g[i];
        m[i] = beta1 * m[i] + (1.0f - beta1) * gi;
        v[i] = beta2 * v[i] + (1.0f - beta2) * gi * gi;
        float upd = m[i] / (sqrtf(v[i]) + eps_t);
        p[i] -= wdd * p[i];
        p[i] -= lrb * upd;
    }
}

/* ------------------------------------------------------------------ MoE */
/* HashMoe::forward CPU path, rust/src/model.rs:187-306: one thread per expert
 * (model.rs:231-270), tokens of expert e in ascending order (model.rs:190-193),
 * pre = b1_e + sum_c xn[t][c] w1[c][e*dff..] (axpy per c, zero x skipped),
 * hidden = silu(pre) = x / (1 + exp(-x)) (model.rs:79-85),
 * out = b2 + sum_j hidden[t][j] w2[e*dff+j] (axpy per j, zero h skipped).
 * route[t] is the expert of token t; outputs are in token order. */
typedef struct {
    const float *xn, *w1, *b1, *w2, *b2, *pre_in, *hid_in, *dout;
    const int32_t* route;
    long T;
    int d, dff, E, e;
    float *out, *pre, *hidden;
    /* backward, per expert */
    float *dw1, *dw2, *db1, *db2, *dxn;
    long* rows;
    long n;
} moe_job;

static float silu_f(float x) { return x / (1.0f + expf(-x)); }

static void moe_rows(moe_job* j) {
    j->n = 0;
    for (long t = 0; t < j->T; ++t)
        if (j->route[t] == j->e) j->rows[j->n++] = t;
}

static void* moe_fwd_thread(void* p) {
    moe_job* j = (moe_job*)p;
    const int d = j->d, dff = j->dff, e = j->e;
    const long ld1 = (long)j->E * dff;
    moe_rows(j);
    for (long i = 0; i < j->n; ++i) memcpy(j->pre + j->rows[i] * dff, j->b1 + (long)e * dff, dff * sizeof(float));
    for (int c = 0; c < d; ++c) {
        const float* w1row = j->w1 + c * ld1 + (long)e * dff;
        for (long i = 0; i < j->n; ++i) {
            const long t = j->rows[i];
            const float xc = j->xn[t * d + c];
            if (xc == 0.0f) continue;
            saxpy(j->pre + t * dff, xc, w1row, dff);
        }
    }
    for (long i = 0; i < j->n; ++i) {
        const long t = j->rows[i];
        for (int q = 0; q < dff; ++q) j->hidden[t * dff + q] = silu_f(j->pre[t * dff + q]);
        memcpy(j->out + t * d, j->b2, d * sizeof(float));
    }
    for (int q = 0; q < dff; ++q) {
        const float* w2row = j->w2 + ((long)e * dff + q) * d;
        for (long i = 0; i < j->n; ++i) {
            const long t = j->rows[i];
            const float h = j->hidden[t * dff + q];
            if (h == 0.0f) continue;
            saxpy(j->out + t * d, h, w2row, d);
        }
    }
    return NULL;
}

static void moe_run(moe_job* jobs, int E, void* (*fn)(void*)) {
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * E);
    for (int e = 0; e < E; ++e) pthread_create(&th[e], NULL, fn, &jobs[e]);
    for (int e = 0; e < E; ++e) pthread_join(th[e], NULL);
    free(th);
}

ORC_API void orc_moe_fwd(const float* xn, const float* w1, const float* b1, const float* w2, const float* b2,
                         const int32_t* route, long T, int d, int dff, int E,
                         float* out, float* pre, float* hidden) {
    moe_job* jobs = (moe_job*)calloc(E, sizeof(moe_job));
    for (int e = 0; e < E; ++e) {
        moe_job* j = &jobs[e];
        j->xn = xn; j->w1 = w1; j->b1 = b1; j->w2 = w2; j->b2 = b2; j->route = route;
        j->T = T; j->d = d; j->dff = dff; j->E = E; j->e = e;
        j->out = out; j->pre = pre; j->hidden = hidden;
        j->rows = (long*)malloc(sizeof(long) * (T > 0 ? T : 1));
    }
    moe_run(jobs, E, moe_fwd_thread);
    for (int e = 0; e < E; ++e) free(jobs[e].rows);
    free(jobs);
}

/* HashMoe::backward CPU path, rust/src/model.rs:365-497 (before its RMSNorm
 * backward): per expert, into the expert's own buffers (model.rs:370-397),
 *   dW2_e[j] += h[t][j] dout[t] (axpy, zero h skipped); db2_e += dout[t];
 *   dpre = dot(dout[t], w2[e*dff+j]); dh = dpre * s (1 + pre (1 - s)), db1_e += dh;
 *   dW1_e[c] += xn[t][c] dh (axpy, zero x skipped); dxn_e[i][c] += dot(dh_i, w1[c][e*dff..]);
 * then merged in expert order (model.rs:466-494).  Gradients are written
 * (the Param::grad buffers are taken to start at zero). */
static void* moe_bwd_thread(void* p) {
    moe_job* j = (moe_job*)p;
    const int d = j->d, dff = j->dff, e = j->e;
    const long ld1 = (long)j->E * dff;
    moe_rows(j);
    const long n = j->n;
    if (n == 0) return NULL;
    float* dpre = (float*)calloc((size_t)n * dff, sizeof(float));
    for (long i = 0; i < n; ++i) {
        const long t = j->rows[i];
        const float* dr = j->dout + t * d;
        for (int q = 0; q < dff; ++q) {
            const float h = j->hid_in[t * dff + q];
            if (h == 0.0f) continue;
            saxpy(j->dw2 + (long)q * d, h, dr, d);
        }
        for (int c = 0; c < d; ++c) j->db2[c] += dr[c];
    }
    for (long i = 0; i < n; ++i) {
        const float* dr = j->dout + j->rows[i] * d;
        for (int q = 0; q < dff; ++q) dpre[i * dff + q] = sdot(dr, j->w2 + ((long)e * dff + q) * d, d);
    }
    for (long i = 0; i < n; ++i) {
        const long t = j->rows[i];
        for (int q = 0; q < dff; ++q) {
            const float pr = j->pre_in[t * dff + q];
            const float sg = 1.0f / (1.0f + expf(-pr));
            const float dh = dpre[i * dff + q] * (sg * (1.0f + pr * (1.0f - sg)));
            j->db1[q] += dh;
            dpre[i * dff + q] = dh;
        }
    }
    for (int c = 0; c < d; ++c) {
        const float* w1row = j->w1 + c * ld1 + (long)e * dff;
        float* gw = j->dw1 + (long)c * dff;
        for (long i = 0; i < n; ++i) {
            const float xc = j->xn[j->rows[i] * d + c];
            if (xc == 0.0f) continue;
            saxpy(gw, xc, dpre + i * dff, dff);
        }
        for (long i = 0; i < n; ++i) j->dxn[i * d + c] += sdot(dpre + i * dff, w1row, dff);
    }
    free(dpre);
    return NULL;
}

ORC_API void orc_moe_bwd(const float* xn, const float* w1, const float* w2, const float* pre,
                         const float* hidden, const int32_t* route, const float* dout,
                         long T, int d, int dff, int E,
                         float* dxn, float* dw1, float* db1, float* dw2, float* db2) {
    moe_job* jobs = (moe_job*)calloc(E, sizeof(moe_job));
    for (int e = 0; e < E; ++e) {
        moe_job* j = &jobs[e];
        j->xn = xn; j->w1 = w1; j->w2 = w2; j->pre_in = pre; j->hid_in = hidden; j->dout = dout;
        j->route = route; j->T = T; j->d = d; j->dff = dff; j->E = E; j->e = e;
        j->rows = (long*)malloc(sizeof(long) * (T > 0 ? T : 1));
        j->dw1 = (float*)calloc((size_t)d * dff, sizeof(float));
        j->dw2 = (float*)calloc((size_t)dff * d, sizeof(float));
        j->db1 = (float*)calloc(dff, sizeof(float));
        j->db2 = (float*)calloc(d, sizeof(float));
        j->dxn = (float*)calloc((size_t)(T > 0 ? T : 1) * d, sizeof(float));
    }
    moe_run(jobs, E, moe_bwd_thread);
    const long ld1 = (long)E * dff;
    memset(dxn, 0, sizeof(float) * T * d);
    memset(dw1, 0, sizeof(float) * d * ld1);
    memset(dw2, 0, sizeof(float) * ld1 * d);
    memset(db1, 0, sizeof(float) * ld1);
    memset(db2, 0, sizeof(float) * d);
    for (int e = 0; e < E; ++e) {
        moe_job* j = &jobs[e];
        for (int q = 0; q < dff; ++q)
            for (int c = 0; c < d; ++c) dw2[((long)e * dff + q) * d + c] += j->dw2[(long)q * d + c];
        for (int c = 0; c < d; ++c)
            for (int q = 0; q < dff; ++q) dw1[c * ld1 + (long)e * dff + q] += j->dw1[(long)c * dff + q];
        for (int q = 0; q < dff; ++q) db1[(long)e * dff + q] += j->db1[q];
        for (int c = 0; c < d; ++c) db2[c] += j->db2[c];
        for (long i = 0; i < j->n; ++i)
            for (int c = 0; c < d; ++c) dxn[j->rows[i] * d + c] += j->dxn[i * d + c];
        free(j->rows); free(j->dw1); free(j->dw2); free(j->db1); free(j->db2); free(j->dxn);
    }
    free(jobs);
}

/* ------------------------------------------------------- cross-entropy */
/* cpu_cross_entropy, rust/src/model.rs:804-844, as one chunk (the reference's
 * per-thread loss partials only regroup the sum): per row lse = max +
 * ln(sum exp(x - max)); loss += lse - x[target]; dlogits = exp(x - lse) / T,
 * then minus 1/T at the target.  Returns the mean loss. */
ORC_API float orc_cross_entropy(const float* logits, const uint32_t* targets, long T, int V, float* dlogits) {
    const float inv = 1.0f / (float)T;
    float l = 0.0f;
    for (long t = 0; t < T; ++t) {
        const float* row = logits + t * V;
        float mx = -INFINITY;
        for (int c = 0; c < V; ++c) mx = fmaxf(mx, row[c]);
        float sum = 0.0f;
        for (int c = 0; c < V; ++c) sum += expf(row[c] - mx);
        const float lse = mx + logf(sum);
        l += lse - row[targets[t]];
        float* dr = dlogits + t * V;
        for (int c = 0; c < V; ++c) dr[c] = expf(row[c] - lse) * inv;
        dr[targets[t]] -= inv;
    }
    return l * inv;
}
