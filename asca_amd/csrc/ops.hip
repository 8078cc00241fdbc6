// Row-wise and element-wise ops around the delta block: RMSNorm fwd/bwd
// (no gain), AdamW with the CPU path's semantics, hash routing with a stable
// expert bucketing, row gather/scatter, and softmax cross-entropy.
//
// All reductions are wave-level butterflies (no atomics), so results are
// deterministic; one wave per row.
#include "common.h"
#include "ops.h"
#include "runtime.h"

namespace asca {

constexpr int ROW_NT = 256;  // 4 rows per block

// ------------------------------------------------------------------ RMSNorm

// rmsnorm_rows (rust/src/tensor.rs:259-270): y = x / sqrt(mean(x^2) + eps).
__global__ __launch_bounds__(ROW_NT) void rmsnorm_k(const float* __restrict__ x, float* __restrict__ y,
                                                   float* __restrict__ inv_out, long rows, int cols, float eps) {
    const long r = (long)blockIdx.x * (ROW_NT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float* xr = x + r * cols;
    float ss = 0.0f;
    for (int c = lane; c < cols; c += 64) ss = fmaf(xr[c], xr[c], ss);
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
    for (int c = lane; c < cols; c += 64) y[r * cols + c] = xr[c] * inv;
    if (inv_out && lane == 0) inv_out[r] = inv;
}

// rmsnorm_rows_backward (rust/src/tensor.rs:282-296):
// dx = inv * (dy - x * inv * mean(dy * x) * inv), mean over the row; with
// `res`, the residual gradient it joins is added (model.rs:769-777).
__global__ __launch_bounds__(ROW_NT) void rmsnorm_bwd_k(const float* __restrict__ x, const float* __restrict__ dy,
                                                       const float* __restrict__ res, float* __restrict__ dx,
                                                       long rows, int cols, float eps) {
    const long r = (long)blockIdx.x * (ROW_NT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float* xr = x + r * cols;
    const float* dr = dy + r * cols;
    float ss = 0.0f, sd = 0.0f;
    for (int c = lane; c < cols; c += 64) {
        ss = fmaf(xr[c], xr[c], ss);
        sd = fmaf(dr[c], xr[c], sd);
    }
    ss = wave_sum(ss);
    sd = wave_sum(sd);
    const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
    const float mean = sd * inv / (float)cols;
    if (res) {
        const float* rr = res + r * cols;
        for (int c = lane; c < cols; c += 64) dx[r * cols + c] = rr[c] + inv * (dr[c] - xr[c] * inv * mean);
    } else {
        for (int c = lane; c < cols; c += 64) dx[r * cols + c] = inv * (dr[c] - xr[c] * inv * mean);
    }
}

// -------------------------------------------------------------------- AdamW

// The element update of AdamW::update's CPU path (rust/src/tensor.rs:444-453),
// operation by operation without contraction (Rust never fuses a multiply
// into an add; HIP's '/' and sqrtf are correctly rounded by default), so the
// results match the CPU bit for bit:
//   m = b1 m + (1-b1) g;  v = b2 v + (1-b2) g g;  upd = m / (sqrt(v) + eps_t)
//   p -= wd p;  p -= lr upd
__global__ __launch_bounds__(256) void adamw_k(float* __restrict__ p, const float* __restrict__ g,
                                              float* __restrict__ m, float* __restrict__ v, long n, float lr,
                                              float b1, float b2, float omb1, float omb2, float eps_t, float wd) {
#pragma clang fp contract(off)
    const long stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float gi = g[i];
        const float mi = b1 * m[i] + omb1 * gi;
        const float vi = b2 * v[i] + omb2 * gi * gi;
        m[i] = mi;
        v[i] = vi;
        const float upd = mi / (sqrtf(vi) + eps_t);
        float pi = p[i];
        pi -= wd * pi;
        pi -= lr * upd;
        p[i] = pi;
    }
}

// ------------------------------------------------------------ hash routing

// hash_route (rust/src/model.rs:69-77), wrapping u32 arithmetic.
ASCA_DEV uint32_t hash_expert(uint32_t id, uint32_t n) {
    uint32_t h = id * 0x9E3779B1u;
    h ^= h >> 15;
    h *= 0x85EBCA6Bu;
    h ^= h >> 13;
    return h % n;
}

constexpr int RT_NT = 256;     // tokens per routing block (one per thread)
constexpr int RT_MAXB = 256;   // buckets (experts, or vocabulary ids)

// Pass 1: bucket of every token and the per-block count of every bucket.
// HASH: bucket = hash_route(id) % E; otherwise the key itself (key < E).
template <bool HASH>
__global__ __launch_bounds__(RT_NT) void route_count_k(const uint32_t* __restrict__ ids, int n, int E,
                                                       int32_t* __restrict__ expert, int32_t* __restrict__ blkcnt) {
    __shared__ int cnt[RT_MAXB];
    const int t = blockIdx.x * RT_NT + threadIdx.x;
    for (int e = threadIdx.x; e < E; e += RT_NT) cnt[e] = 0;
    __syncthreads();
    if (t < n) {
        // keys >= E wrap (memory safety); callers pass keys < E
        const int e = (int)(HASH ? hash_expert(ids[t], (uint32_t)E) : ids[t] % (uint32_t)E);
        expert[t] = e;
        atomicAdd(&cnt[e], 1);  // integer counts: order-independent
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += RT_NT) blkcnt[blockIdx.x * E + e] = cnt[e];
}

// Pass 2 (one block, thread e = bucket): bucket offsets and, per block, where
// its tokens of each bucket start; blkcnt is rewritten in place as the starts.
__global__ __launch_bounds__(RT_MAXB) void route_scan_k(int nblk, int E, int32_t* __restrict__ blkcnt,
                                                        int32_t* __restrict__ offsets) {
    __shared__ int wtot[RT_MAXB / 64];
    const int e = threadIdx.x, lane = e & 63, w = e >> 6;
    int total = 0;
    if (e < E)
        for (int b = 0; b < nblk; ++b) total += blkcnt[b * E + e];
    int incl = total;  // inclusive scan inside the wave
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) {
        const int o = __shfl_up(incl, s, 64);
        if (lane >= s) incl += o;
    }
    if (lane == 63) wtot[w] = incl;
    __syncthreads();
    for (int ww = 0; ww < w; ++ww) incl += wtot[ww];
    const int base = incl - total;
    if (e < E) {
        offsets[e] = base;
        if (e == E - 1) offsets[E] = incl;
        int run = base;
        for (int b = 0; b < nblk; ++b) {
            const int c = blkcnt[b * E + e];
            blkcnt[b * E + e] = run;
            run += c;
        }
    }
}

// Pass 3: stable placement -- a token's rank among the earlier tokens of its
// block in the same bucket comes from wave ballots, so every bucket lists its
// tokens in ascending order, as model.rs:190-193 builds them.
__global__ __launch_bounds__(RT_NT) void route_place_k(int n, int E, const int32_t* __restrict__ expert,
                                                       const int32_t* __restrict__ blkstart,
                                                       int32_t* __restrict__ perm) {
    __shared__ unsigned char wcnt[RT_NT / 64][RT_MAXB];  // tokens per (wave, bucket), <= 64
    const int t = blockIdx.x * RT_NT + threadIdx.x;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int my = t < n ? expert[t] : -1;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int rank = 0;
    for (int e = 0; e < E; ++e) {
        const uint64_t mask = __ballot(my == e);
        if (my == e) rank = __popcll(mask & below);
        if (lane == 0) wcnt[w][e] = (unsigned char)__popcll(mask);
    }
    __syncthreads();
    if (t < n) {
        int before = 0;
        for (int ww = 0; ww < w; ++ww) before += wcnt[ww][my];
        perm[blkstart[blockIdx.x * E + my] + before + rank] = t;
    }
}

// Counting sort of n tokens into E <= 256 buckets (stable).  ws: nblk * E ints.
int bucket_launch(bool hash, const uint32_t* ids, int n, int E, int32_t* expert, int32_t* perm, int32_t* offsets,
                  void* ws, hipStream_t st) {
    const int nblk = (n + RT_NT - 1) / RT_NT;
    int32_t* blk = reinterpret_cast<int32_t*>(ws);
    int rc;
    if (n > 0) {
        rc = pre_launch("route_count");
        if (rc) return rc;
        if (hash)
            hipLaunchKernelGGL(route_count_k<true>, dim3(nblk), dim3(RT_NT), 0, st, ids, n, E, expert, blk);
        else
            hipLaunchKernelGGL(route_count_k<false>, dim3(nblk), dim3(RT_NT), 0, st, ids, n, E, expert, blk);
        rc = post_launch("route_count");
        if (rc) return rc;
    }
    rc = pre_launch("route_scan");
    if (rc) return rc;
    hipLaunchKernelGGL(route_scan_k, dim3(1), dim3(RT_MAXB), 0, st, nblk, E, blk, offsets);
    rc = post_launch("route_scan");
    if (rc || n == 0) return rc;
    rc = pre_launch("route_place");
    if (rc) return rc;
    hipLaunchKernelGGL(route_place_k, dim3(nblk), dim3(RT_NT), 0, st, n, E, expert, blk, perm);
    return post_launch("route_place");
}

// ------------------------------------------------------------ gather/scatter

// dst[r] = src[idx[r]] (gather_rows_f32, rust/kernels/asca.cu:576-584), or with
// SCATTER dst[idx[r]] = src[r] (asca.cu:586-594; indices unique).
template <bool SCATTER, bool VEC>
__global__ __launch_bounds__(ROW_NT) void rows_copy_k(const float* __restrict__ src, const int32_t* __restrict__ idx,
                                                     long n, int cols, float* __restrict__ dst) {
    const long r = (long)blockIdx.x * (ROW_NT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= n) return;
    const long sr = SCATTER ? r : (long)idx[r];
    const long dr = SCATTER ? (long)idx[r] : r;
    if constexpr (VEC) {
        const float4* s4 = reinterpret_cast<const float4*>(src + sr * cols);
        float4* d4 = reinterpret_cast<float4*>(dst + dr * cols);
        for (int c = lane; c < cols / 4; c += 64) d4[c] = s4[c];
    } else {
        for (int c = lane; c < cols; c += 64) dst[dr * cols + c] = src[sr * cols + c];
    }
}

// ------------------------------------------------------------ cross-entropy

// Per row t: lse = max + ln(sum exp(x - max)); loss_t = lse - x[target];
// dlogits = exp(x - lse) / T, minus 1/T at the target (cpu_cross_entropy,
// rust/src/model.rs:804-844).
__global__ __launch_bounds__(ROW_NT) void cross_entropy_k(const float* __restrict__ logits,
                                                         const uint32_t* __restrict__ targets, long T, int V,
                                                         float inv_t, float* __restrict__ dlogits,
                                                         float* __restrict__ losses) {
    const long t = (long)blockIdx.x * (ROW_NT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= T) return;
    const float* row = logits + t * V;
    float mx = -INFINITY;
    for (int c = lane; c < V; c += 64) mx = fmaxf(mx, row[c]);
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) mx = fmaxf(mx, __shfl_xor(mx, s, 64));
    float sum = 0.0f;
    for (int c = lane; c < V; c += 64) sum += expf(row[c] - mx);
    sum = wave_sum(sum);
    const float lse = mx + logf(sum);
    const uint32_t tg = targets[t];
    if (lane == 0) losses[t] = tg < (uint32_t)V ? lse - row[tg] : 0.0f;
    float* drow = dlogits + t * V;
    for (int c = lane; c < V; c += 64) {
        float pr = expf(row[c] - lse) * inv_t;
        if ((uint32_t)c == tg) pr -= inv_t;
        drow[c] = pr;
    }
}

}  // namespace asca

using namespace asca;

static unsigned row_blocks(long rows) { return (unsigned)((rows + (ROW_NT / 64) - 1) / (ROW_NT / 64)); }

int asca::rmsnorm_bwd_launch(const float* x, const float* dy, const float* res, float* dx, long rows, int cols,
                             float eps, hipStream_t st) {
    if (rows == 0 || cols == 0) return ASCA_OK;
    int rc = pre_launch("rmsnorm_bwd");
    if (rc) return rc;
    hipLaunchKernelGGL(rmsnorm_bwd_k, dim3(row_blocks(rows)), dim3(ROW_NT), 0, st, x, dy, res, dx, rows, cols, eps);
    return post_launch("rmsnorm_bwd");
}

extern "C" {

int asca_rmsnorm(const float* x, float* y, float* inv, long rows, int cols, float eps, void* stream) {
    if (rows < 0 || cols < 0) return fail(ASCA_ERR_INVALID, "negative shape");
    if (rows == 0 || cols == 0) return ASCA_OK;
    if (!x || !y) return fail(ASCA_ERR_INVALID, "null pointer in asca_rmsnorm");
    int rc = pre_launch("rmsnorm");
    if (rc) return rc;
    hipLaunchKernelGGL(rmsnorm_k, dim3(row_blocks(rows)), dim3(ROW_NT), 0, as_stream(stream), x, y, inv, rows, cols,
                       eps);
    return post_launch("rmsnorm");
}

int asca_rmsnorm_bwd(const float* x, const float* dy, float* dx, long rows, int cols, float eps, void* stream) {
    if (rows < 0 || cols < 0) return fail(ASCA_ERR_INVALID, "negative shape");
    if (rows == 0 || cols == 0) return ASCA_OK;
    if (!x || !dy || !dx) return fail(ASCA_ERR_INVALID, "null pointer in asca_rmsnorm_bwd");
    return rmsnorm_bwd_launch(x, dy, nullptr, dx, rows, cols, eps, as_stream(stream));
}

int asca_adamw_scalars(float lr, float beta1, float beta2, float eps, float wd, uint32_t step, float* out) {
#pragma clang fp contract(off)
    if (!out) return fail(ASCA_ERR_INVALID, "null output pointer");
    if (step == 0 || step > 0x7fffffffu) return fail(ASCA_ERR_INVALID, "adamw step %u outside 1..2^31-1", step);
    // f32::powi with a run-time exponent is binary exponentiation
    auto powi = [](float a, int b) {
        float r = 1.0f;
        for (;;) {
            if (b & 1) r *= a;
            b /= 2;
            if (b == 0) break;
            a *= a;
        }
        return r;
    };
    const float bc1 = 1.0f - powi(beta1, (int)step);
    const float bc2 = 1.0f - powi(beta2, (int)step);
    out[0] = lr * sqrtf(bc1 / bc2);
    out[1] = eps * sqrtf(bc2);
    out[2] = lr * wd;
    return ASCA_OK;
}

int asca_adamw(float* p, const float* g, float* m, float* v, long n, float lr, float beta1, float beta2,
               float eps_t, float wd, void* stream) {
    if (n < 0) return fail(ASCA_ERR_INVALID, "negative size");
    if (n == 0) return ASCA_OK;
    if (!p || !g || !m || !v) return fail(ASCA_ERR_INVALID, "null pointer in asca_adamw");
    int rc = pre_launch("adamw");
    if (rc) return rc;
    long blocks = (n + 255) / 256;
    const long cap = (long)(cu_count() > 0 ? cu_count() : 256) * 16;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL(adamw_k, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), p, g, m, v, n, lr, beta1,
                       beta2, 1.0f - beta1, 1.0f - beta2, eps_t, wd);
    return post_launch("adamw");
}

int asca_hash_route_ws_bytes(int n, int n_experts, size_t* bytes) {
    if (!bytes) return fail(ASCA_ERR_INVALID, "null output pointer");
    if (n < 0 || n_experts < 1 || n_experts > RT_MAXB)
        return fail(ASCA_ERR_UNSUPPORTED, "bucketing: n=%d buckets=%d (1..%d buckets)", n, n_experts, RT_MAXB);
    const long nblk = (n + RT_NT - 1) / RT_NT;
    *bytes = (size_t)(nblk > 0 ? nblk : 1) * n_experts * sizeof(int32_t);
    return ASCA_OK;
}

static int bucket_entry(bool hash, const uint32_t* ids, int n, int n_experts, int32_t* expert, int32_t* perm,
                        int32_t* offsets, void* ws, void* stream) {
    size_t wsb = 0;
    int rc = asca_hash_route_ws_bytes(n, n_experts, &wsb);
    if (rc) return rc;
    if (!offsets) return fail(ASCA_ERR_INVALID, "null offsets");
    if (n > 0 && (!ids || !expert || !perm || !ws)) return fail(ASCA_ERR_INVALID, "null pointer in bucketing");
    return bucket_launch(hash, ids, n, n_experts, expert, perm, offsets, ws, as_stream(stream));
}

int asca_hash_route(const uint32_t* ids, int n, int n_experts, int32_t* expert, int32_t* perm, int32_t* offsets,
                    void* ws, void* stream) {
    return bucket_entry(true, ids, n, n_experts, expert, perm, offsets, ws, stream);
}

int asca_bucket_keys(const uint32_t* keys, int n, int n_buckets, int32_t* bucket, int32_t* perm, int32_t* offsets,
                     void* ws, void* stream) {
    return bucket_entry(false, keys, n, n_buckets, bucket, perm, offsets, ws, stream);
}

static int rows_copy(bool scatter, const float* src, const int32_t* idx, long n, int cols, float* dst, void* stream) {
    if (n < 0 || cols < 0) return fail(ASCA_ERR_INVALID, "negative shape");
    if (n == 0 || cols == 0) return ASCA_OK;
    if (!src || !idx || !dst) return fail(ASCA_ERR_INVALID, "null pointer in row gather/scatter");
    const char* name = scatter ? "scatter_rows" : "gather_rows";
    int rc = pre_launch(name);
    if (rc) return rc;
    const bool vec = cols % 4 == 0 && ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
    const hipStream_t st = as_stream(stream);
    if (scatter) {
        if (vec) hipLaunchKernelGGL((rows_copy_k<true, true>), dim3(row_blocks(n)), dim3(ROW_NT), 0, st, src, idx, n, cols, dst);
        else hipLaunchKernelGGL((rows_copy_k<true, false>), dim3(row_blocks(n)), dim3(ROW_NT), 0, st, src, idx, n, cols, dst);
    } else {
        if (vec) hipLaunchKernelGGL((rows_copy_k<false, true>), dim3(row_blocks(n)), dim3(ROW_NT), 0, st, src, idx, n, cols, dst);
        else hipLaunchKernelGGL((rows_copy_k<false, false>), dim3(row_blocks(n)), dim3(ROW_NT), 0, st, src, idx, n, cols, dst);
    }
    return post_launch(name);
}

int asca_gather_rows(const float* src, const int32_t* idx, long n, int cols, float* dst, void* stream) {
    return rows_copy(false, src, idx, n, cols, dst, stream);
}

int asca_scatter_rows(const float* src, const int32_t* idx, long n, int cols, float* dst, void* stream) {
    return rows_copy(true, src, idx, n, cols, dst, stream);
}

int asca_cross_entropy(const float* logits, const uint32_t* targets, long T, int V, float* dlogits, float* losses,
                       void* stream) {
    if (T < 0 || V <= 0) return fail(ASCA_ERR_INVALID, "bad shape T=%ld V=%d", T, V);
    if (T == 0) return ASCA_OK;
    if (!logits || !targets || !dlogits || !losses) return fail(ASCA_ERR_INVALID, "null pointer in asca_cross_entropy");
    int rc = pre_launch("cross_entropy");
    if (rc) return rc;
    hipLaunchKernelGGL(cross_entropy_k, dim3(row_blocks(T)), dim3(ROW_NT), 0, as_stream(stream), logits, targets, T, V,
                       1.0f / (float)T, dlogits, losses);
    return post_launch("cross_entropy");
}

}  // extern "C"
