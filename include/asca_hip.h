/*
 * asca_hip.h -- C ABI of libasca_hip.so, the MI355X (gfx950) backend of the
 * ASCA gated delta-rule hot path.
 *
 * It replaces the reference crate's CUDA FFI module (rust/src/cuda/sys.rs:33-65,
 * hand-bound CUDA driver API) plus the PTX kernels it launches
 * (rust/kernels/asca.cu), under the unchanged operator API of
 * rust/src/cuda/mod.rs (`Gpu::delta_scan`, `Gpu::delta_bwd_dev`, ...).
 *
 * Conventions
 *   - Every function returns an int status: 0 (ASCA_OK) or a positive error
 *     code; none aborts.  asca_last_error() gives the message of the calling
 *     thread's last failure (rust/src/cuda/sys.rs:68-70 maps CUresult the same way).
 *   - Tensor arguments are device pointers to row-major f32 data unless stated.
 *     The caller owns every buffer it passes.
 *   - `stream` is an opaque hipStream_t (NULL = the null stream).  Entry points
 *     that take a stream are asynchronous; synchronise before reading results on
 *     the host.  The reference synchronises after every op (cuCtxSynchronize).
 *   - Row layout follows the reference: row r = b*T + t of a (B*T, H*dh) matrix
 *     holds token t of sequence b, head h in columns h*dh .. h*dh+dh-1
 *     (rust/kernels/asca.cu:256-263, rust/src/delta.rs:118-120).
 */
#ifndef ASCA_HIP_H
#define ASCA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ASCA_API __attribute__((visibility("default")))

enum {
    ASCA_OK = 0,
    ASCA_ERR_INVALID = 1,      /* bad argument (shape, null pointer, range)      */
    ASCA_ERR_HIP = 2,          /* a HIP runtime call failed                       */
    ASCA_ERR_UNSUPPORTED = 3,  /* shape or device this build does not handle      */
    ASCA_ERR_NOT_INIT = 4,     /* asca_init has not succeeded                      */
    ASCA_ERR_INJECTED = 5,     /* failure injected by asca_fail_after             */
    ASCA_ERR_OOM = 6,          /* device allocation failed                        */
    ASCA_ERR_NO_DEVICE = 7,    /* no HIP device present                           */
    ASCA_ERR_PARTIAL_UPDATE = 8 /* asca_model_train_step: the optimiser step failed
                                  after updating some tensors (see there)        */
};

/* ------------------------------------------------------------ runtime ---- */

/* Message of the calling thread's last error ("" if none). */
ASCA_API const char* asca_last_error(void);

/* Replaces cuInit + cuDeviceGet + cuCtxCreate_v2 (sys.rs:34-44) as used by
 * Gpu::init (rust/src/cuda/mod.rs:177-237).  Fails unless `device` is gfx950. */
ASCA_API int asca_init(int device);

/* Replaces cuDeviceGetCount-style probing behind cuda::available() (mod.rs:1508). */
ASCA_API int asca_device_count(int* n);

/* Replaces cuDeviceGetName + cuDeviceGetAttribute(SM count) used by
 * cuda::describe() (mod.rs:1494-1530): "name (arch, N CUs)". */
ASCA_API int asca_describe(char* buf, int len);

/* Replaces cuMemAlloc_v2 / cuMemFree_v2 (sys.rs:47-48) behind DevBuf's
 * size-class pool (mod.rs:100-174): sizes round up to a power of two and
 * freed blocks are recycled, never returned to HIP until asca_pool_release. */
ASCA_API int asca_alloc(void** ptr, size_t bytes);
ASCA_API int asca_free(void* ptr);
ASCA_API int asca_pool_release(void);

/* Replaces cuMemcpyHtoD_v2 / cuMemcpyDtoH_v2 (sys.rs:49-50) behind
 * DevBuf::upload/download (mod.rs:126-157).  Synchronous; counted in
 * asca_stats exactly as H2D_BYTES / D2H_BYTES are (mod.rs:25-27). */
ASCA_API int asca_h2d(void* dst, const void* src, size_t bytes);
ASCA_API int asca_d2h(void* dst, const void* src, size_t bytes);
/* Device-to-device copy on `stream` (no reference counterpart: the reference
 * never copies on the device). */
ASCA_API int asca_d2d(void* dst, const void* src, size_t bytes, void* stream);

/* Replaces cuMemsetD32_v2 (sys.rs:51). */
ASCA_API int asca_memset32(void* dst, uint32_t value, size_t count, void* stream);

/* Replaces cuCtxSynchronize (sys.rs:45). */
ASCA_API int asca_sync(void);
ASCA_API int asca_stream_sync(void* stream);

/* Traffic and launch counters: H2D_BYTES, D2H_BYTES, LAUNCHES and
 * reset_stats() of rust/src/cuda/mod.rs:25-33. */
ASCA_API int asca_stats(uint64_t* h2d, uint64_t* d2h, uint64_t* launches);
ASCA_API int asca_reset_stats(void);

/* Fault injection for the CPU-fallback paths (delta.rs:227-240, 640-647): the
 * n-th kernel launch from now (0 = the next one) fails with ASCA_ERR_INJECTED
 * without launching; -1 disables.  ASCA_FAIL_LAUNCH=n in the environment sets
 * it at asca_init.  No reference counterpart. */
ASCA_API int asca_fail_after(int64_t n);

/* Streams (default priority, non-blocking) and events for timing.  No
 * reference counterpart: the reference only uses the null stream. */
ASCA_API int asca_stream_create(void** stream);
ASCA_API int asca_stream_destroy(void* stream);
ASCA_API int asca_event_create(void** ev);
ASCA_API int asca_event_destroy(void* ev);
ASCA_API int asca_event_record(void* ev, void* stream);
/* Waits for `stop`, then returns the time between the two events in ms. */
ASCA_API int asca_event_elapsed_ms(float* ms, void* start, void* stop);

/* Diagnostic: runs one wave through the lane-exchange primitives the kernels
 * use (DPP quad_perm xor1/xor2, row_half_mirror, row_mirror, row_ror:8,
 * permlane32_swap, permlane16_swap, full-wave sum) on x[lane] = lane and
 * y[lane] = 100 + lane, then one v_mfma_f32_16x16x4_f32 on small-integer
 * operands a[lane] = (7 lane) % 13 - 6, b[lane] = (5 lane) % 11 - 5 (rows 10-13:
 * its four result registers), then the row_shr prefix products over 8 and 2
 * lanes of z[lane] = 2^((3 lane) % 5 - 2) (rows 14, 15), and copies 16 x 64
 * floats to host_out (row c = result c per lane).  No reference counterpart. */
ASCA_API int asca_selftest_wave(float* host_out);

/* Plain streaming device copy of n floats (n % 4 == 0, 16-byte aligned
 * buffers).  The known-size kernel against which HBM traffic counters are
 * calibrated.  No reference counterpart. */
ASCA_API int asca_copy_f32(float* dst, const float* src, size_t n, void* stream);

/* ---------------------------------------------------------------- rng --- */
/* Host-side restatement of the reference's input generator Rng
 * (rust/src/tensor.rs:299-337): xorshift128+ seeded as Rng::new(seed)
 * (:307-311), next_u64 (:313-320), Box-Muller normal() in f32 (:328-332).
 * state[2] carries the stream between calls. */
ASCA_API void asca_rng_seed(uint64_t seed, uint64_t* state);
ASCA_API void asca_rng_u64(uint64_t* state, uint64_t* out, size_t n);
/* out[i] = offset + normal() * scale */
ASCA_API void asca_rng_normal(uint64_t* state, float* out, size_t n, float scale, float offset);

/* --------------------------------------------------- delta rule (recurrent) */

/* Bytes of the workspace a delta forward leaves for its backward: one dh-vector
 * per token-head (B*T*H*dh floats: S_{t-1}^T k_t; at dh = 64 the u_t rows, with
 * T rounded up to a multiple of 16) and state checkpoints every C steps plus the final state
 * (B*H*(ceil(T/C)+1)*dh*dh floats; C depends on dh, 32 at dh = 64); at dh = 64
 * also a record of 1344 floats per 16-step block and unit
 * (B*H*ceil(T/16)*1344 floats: the block's Gram products, triangular factors and
 * gate vectors).  It replaces the full state history DeltaDev.states of
 * rust/src/cuda/mod.rs:1274-1275,1386-1397 ((T+1)*dh*dh floats per unit).
 * dh may be 1..128.  The forward writes the workspace and the backwards only
 * read it, so several backwards may use one forward's workspace at once. */
ASCA_API int asca_delta_ws_bytes(int B, int T, int H, int dh, size_t* bytes);

/* Forward recurrence of the gated delta rule for all (sequence, head) units,
 * S_0 = 0:  sk_t = S_{t-1}^T k_t;  u_t = beta_t (v_t - alpha_t sk_t);
 *           S_t = alpha_t S_{t-1} + k_t u_t^T;  o_t = S_t^T q_t.
 * Replaces Gpu::delta_scan (rust/src/cuda/mod.rs:1253-1321) and kernel
 * delta_fwd_batch_f32 (rust/kernels/asca.cu:256-317); same math as
 * DeltaBlock::scan_cpu (rust/src/delta.rs:244-334).
 *   q, k, v : (B*T, H*dh), q and k already L2-normalised per head
 *   alpha, beta : (B*T, H)
 *   o : (B*T, H*dh) output
 *   ws : asca_delta_ws_bytes(B,T,H,dh) bytes, kept for asca_delta_bwd_* (which
 *        read it and never write it) */
ASCA_API int asca_delta_fwd(const float* q, const float* k, const float* v,
                            const float* alpha, const float* beta, float* o, void* ws,
                            int B, int T, int H, int dh, void* stream);

/* BPTT of the recurrence, raw per-head gradients (no L2-norm or sigmoid
 * backward): dq, dk, dv (B*T, H*dh) and dalpha, dbeta (B*T, H).  Same math as
 * the per-(head, sequence) loop of DeltaBlock::bptt_cpu
 * (rust/src/delta.rs:475-572).  Inputs are those of the matching
 * asca_delta_fwd plus d_o (B*T, H*dh); ws must be that call's workspace. */
ASCA_API int asca_delta_bwd_raw(const float* q, const float* k, const float* v,
                                const float* alpha, const float* beta, const float* d_o,
                                const void* ws, float* dq, float* dk, float* dv,
                                float* dalpha, float* dbeta,
                                int B, int T, int H, int dh, void* stream);

/* BPTT with the L2-norm backward of q, k and the sigmoid backward of the gates
 * fused in: the drop-in for Gpu::delta_bwd_dev (rust/src/cuda/mod.rs:1328-1382)
 * and kernel delta_bwd_f32 (rust/kernels/asca.cu:340-485); same results as
 * DeltaBlock::bptt_cpu including its tail (rust/src/delta.rs:589-612).
 *   qnorm, knorm : (B*T, H) norms saved by the forward's L2 normalisation
 *   d_qkv : (B*T, 3*H*dh) = [dq | dk | dv];  d_gate : (B*T, 2*H) = [dalpha | dbeta]
 *   (logit gradients). */
ASCA_API int asca_delta_bwd_fused(const float* q, const float* k, const float* v,
                                  const float* alpha, const float* beta,
                                  const float* qnorm, const float* knorm, const float* d_o,
                                  const void* ws, float* d_qkv, float* d_gate,
                                  int B, int T, int H, int dh, void* stream);

/* Materialise the full state history the reference keeps in DeltaDev.states:
 * for unit u = h*B + b, (T+1) states of dh*dh floats (S before every step, then
 * the final state), row-major S[a][i].  Replaces DeltaDev::download_states
 * (rust/src/cuda/mod.rs:1473-1479), by recomputation.  states is a device
 * buffer of H*B*(T+1)*dh*dh floats. */
ASCA_API int asca_delta_states(const float* q, const float* k, const float* v,
                               const float* alpha, const float* beta, float* states,
                               int B, int T, int H, int dh, void* stream);

/* One decode step for n_seq independent sequences: the state math of
 * DeltaBlock::step (rust/src/delta.rs:356-407) -- per head, q and k of the qkv
 * row are L2-normalised (x * 1/max(|x|, 1e-8)), alpha = sigmoid(gate[h]),
 * beta = sigmoid(gate[H+h]), sk = S^T k, u = beta (v - alpha sk),
 * S = alpha S + k u^T, o = S^T q.  The reference has no GPU decode and caps dh
 * at 64 (delta.rs:361-362); here 1 <= dh <= 128.
 *   states : (n_seq, H, dh, dh) row-major S[a][i], updated in place
 *   qkv    : (n_seq, 3*H*dh) rows of x.w_qkv + b_qkv;  gate : (n_seq, 2*H) logits
 *   o      : (n_seq, H*dh) output */
ASCA_API int asca_delta_decode_step(float* states, const float* qkv, const float* gate, float* o,
                                    int n_seq, int H, int dh, void* stream);

/* ------------------------------------------------------- row operations -- */

/* Row-wise RMSNorm without gain: y = x / sqrt(mean(x^2) + eps) per row of a
 * (rows, cols) matrix; inv (rows, may be NULL) receives 1/rms.  Replaces
 * Gpu::rmsnorm (rust/src/cuda/mod.rs:911-939) and kernel rmsnorm_f32
 * (rust/kernels/asca.cu:198-215); CPU semantics rmsnorm_rows
 * (rust/src/tensor.rs:251-270).  The model uses eps = 1e-6 (model.rs:14). */
ASCA_API int asca_rmsnorm(const float* x, float* y, float* inv, long rows, int cols, float eps,
                          void* stream);

/* RMSNorm backward: dx = inv (dy - x inv mean(dy x inv)) per row.  Replaces
 * Gpu::rmsnorm_bwd (mod.rs:1122-1153), kernel rmsnorm_bwd_f32 (asca.cu:217-242);
 * CPU semantics rmsnorm_rows_backward (tensor.rs:272-297). */
ASCA_API int asca_rmsnorm_bwd(const float* x, const float* dy, float* dx, long rows, int cols, float eps,
                              void* stream);

/* Softmax cross-entropy with its backward, per row t of (T, V) logits:
 * losses[t] = lse_t - logits[t][target_t] (0 for a target >= V), dlogits =
 * softmax / T minus 1/T at the target.  Replaces Gpu::cross_entropy_bwd
 * (mod.rs:945-997) and kernel cross_entropy_bwd_f32 (asca.cu:490-548); CPU
 * semantics cpu_cross_entropy (rust/src/model.rs:804-844).  The mean loss is
 * the sum of losses times 1/T (host side, as the reference does). */
ASCA_API int asca_cross_entropy(const float* logits, const uint32_t* targets, long T, int V,
                                float* dlogits, float* losses, void* stream);

/* dst[r] = src[idx[r]] for r < n, rows of `cols` floats.  Replaces
 * Gpu::gather_rows / gather_raw (mod.rs:401-424,1156-1188) and kernel
 * gather_rows_f32 (asca.cu:576-584).  idx is a device int32 array. */
ASCA_API int asca_gather_rows(const float* src, const int32_t* idx, long n, int cols, float* dst,
                              void* stream);

/* dst[idx[r]] = src[r] for r < n (indices distinct).  Replaces
 * Gpu::scatter_rows / scatter_raw (mod.rs:426-448,1190-1222) and kernel
 * scatter_rows_f32 (asca.cu:586-594). */
ASCA_API int asca_scatter_rows(const float* src, const int32_t* idx, long n, int cols, float* dst,
                               void* stream);

/* out[c] (+)= sum over rows of X[r][c] (accumulate != 0 adds to out): the bias
 * gradient, colsum_raw of rust/src/cuda/mod.rs:642-669.  Deterministic (row
 * slices summed in a fixed order).  The slices' partial sums live in
 * stream-ordered scratch on `stream` (hipMallocAsync / hipFreeAsync), so calls
 * on different streams never share it. */
ASCA_API int asca_colsum(const float* X, long rows, int cols, float* out, int accumulate, void* stream);
/* asca_colsum with the partial sums in a caller workspace of at least
 * asca_colsum_ws_bytes(rows, cols) bytes (no allocation; a workspace must not
 * be shared by calls that overlap).  No reference counterpart: colsum_raw
 * draws its scratch from the crate's pool. */
ASCA_API int asca_colsum_ws_bytes(long rows, int cols, size_t* bytes);
ASCA_API int asca_colsum_ws(const float* X, long rows, int cols, float* out, int accumulate, void* ws,
                            size_t ws_bytes, void* stream);

/* ----------------------------------------------------------------- AdamW -- */

/* The per-step scalars of AdamW::update (rust/src/tensor.rs:392-402), in f32
 * exactly as the CPU computes them, for step s >= 1 (the counter after its
 * increment; the reference counts steps per parameter tensor):
 *   out[0] = lr * sqrt((1 - beta1^s) / (1 - beta2^s))   (bias-corrected lr)
 *   out[1] = eps * sqrt(1 - beta2^s)                    (eps_t)
 *   out[2] = lr * wd                                    (decoupled decay) */
ASCA_API int asca_adamw_scalars(float lr, float beta1, float beta2, float eps, float wd, uint32_t step,
                                float* out);

/* One AdamW update of n parameters in place, moments m, v resident on the
 * device; lr, eps_t, wd as produced by asca_adamw_scalars.  Replaces
 * Gpu::adamw_update / adamw_resident (mod.rs:1003-1119) with the element
 * update of the CPU path (tensor.rs:444-453), bit-exact to it:
 *   m = b1 m + (1-b1) g;  v = b2 v + (1-b2) g g;  p -= wd p;
 *   p -= lr m / (sqrt(v) + eps_t).
 * (The reference's adamw_f32 kernel, asca.cu:551-570, scales the decay by lr
 * a second time; the CPU path is the one followed here.) */
ASCA_API int asca_adamw(float* p, const float* g, float* m, float* v, long n, float lr, float beta1,
                        float beta2, float eps_t, float wd, void* stream);

/* ----------------------------------------------------------- hash routing -- */

/* Workspace bytes for asca_hash_route / asca_bucket_keys (n tokens, 1..256 buckets). */
ASCA_API int asca_hash_route_ws_bytes(int n, int n_experts, size_t* bytes);

/* Expert of every token, expert = hash_route(id) % n_experts with the
 * reference's wrapping u32 finaliser (rust/src/model.rs:69-77), and the
 * buckets of HashMoe::forward (model.rs:190-193) as CSR: perm lists the tokens
 * of expert 0 in ascending order, then expert 1, ...; offsets[e]..offsets[e+1]
 * bound expert e (offsets has n_experts + 1 entries).  Bit-exact and
 * deterministic.  ids: device u32 (n); expert, perm: device int32 (n). */
ASCA_API int asca_hash_route(const uint32_t* ids, int n, int n_experts, int32_t* expert, int32_t* perm,
                             int32_t* offsets, void* ws, void* stream);

/* The same stable bucketing keyed by the value itself (bucket = key, keys <
 * n_buckets <= 256; larger keys wrap modulo n_buckets): tokens grouped by id,
 * the order in which Model::backward accumulates the embedding gradient
 * (rust/src/model.rs:782-789).  Workspace as asca_hash_route_ws_bytes. */
ASCA_API int asca_bucket_keys(const uint32_t* keys, int n, int n_buckets, int32_t* bucket, int32_t* perm,
                              int32_t* offsets, void* ws, void* stream);

/* ------------------------------------------------------------------ GEMM -- */

/* C = alpha op(A) op(B) + bias (per column, may be NULL) + beta C, f32 on the
 * matrix cores; op(A) = A (M x K, lda) or A^T (trans_a: A stored K x M),
 * op(B) = B (K x N, ldb) or B^T (trans_b: B stored N x K).  Column/row offsets
 * into a wider matrix are expressed by pointer and leading dimension.
 * Replaces Gpu::matmul / matmul_ta / matmul_raw / matmul_ta_raw /
 * matmul_ld_raw / matmul_ta_ld_raw / matmul_tb_raw (rust/src/cuda/mod.rs:286-521,
 * 671-743) with kernels matmul_f32 / matmul_ta_f32 / matmul_ld_f32
 * (asca.cu:14-141); CPU semantics Mat::matmul / matmul_ta / matmul_t
 * (rust/src/tensor.rs:91-201).  Deterministic: when the output has too few
 * tiles to fill the device, K is split and the partial products are summed in
 * a fixed order; the partials live in stream-ordered scratch on `stream`
 * (hipMallocAsync / hipFreeAsync), so calls on different streams never share
 * them. */
ASCA_API int asca_gemm(int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A, long lda,
                       const float* B, long ldb, float beta, float* C, long ldc, const float* bias,
                       void* stream);
/* asca_gemm with the split-K partials in a caller workspace of at least
 * asca_gemm_ws_bytes(...) bytes (0 when the product does not split): no
 * allocation and the same results bit for bit; a workspace must not be shared
 * by calls that overlap.  No reference counterpart: matmul_raw draws its
 * buffers from the crate's pool (rust/src/cuda/mod.rs:100-174). */
ASCA_API int asca_gemm_ws_bytes(int trans_a, int trans_b, int M, int N, int K, size_t* bytes);
/* asca_gemm that allocates nothing, for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No reference counterpart.  The split-K partials live in a
 * static 32 MiB device array that every device the library runs on holds
 * until the process ends: the most the split-K partials of any product take
 * on gfx950 (2 * 256 CUs output tiles of 128 x 128 floats), so every product
 * fits; a larger need would be refused with ASCA_ERR_INVALID (asca_gemm_ws
 * takes any size).  The partials are written in
 * full before they are read (nothing needs clearing), and the results are the
 * bits of asca_gemm.  All calls on one device share the array: calls that
 * overlap on one device (concurrent streams or threads) race. */
ASCA_API int asca_gemm_noalloc(int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A,
                               long lda, const float* B, long ldb, float beta, float* C, long ldc,
                               const float* bias, void* stream);
ASCA_API int asca_gemm_ws(int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A, long lda,
                          const float* B, long ldb, float beta, float* C, long ldc, const float* bias, void* ws,
                          size_t ws_bytes, void* stream);

/* ------------------------------------------------------------------- MoE -- */

/* HashMoE forward on normalised input xn (T x d), tokens bucketed by
 * asca_hash_route (perm, offsets): per expert e,
 *   pre = xn[rows_e] w1[:, e*d_ff:(e+1)*d_ff] + b1[e*d_ff..];  hidden = silu(pre)
 *   out[rows_e] = hidden w2[e*d_ff:(e+1)*d_ff, :] + b2
 * as Gpu::moe_forward_dev (rust/src/cuda/mod.rs:523-607) over the CPU
 * semantics of HashMoe::forward (rust/src/model.rs:187-306).  w1 (d x E*d_ff),
 * b1 (E*d_ff), w2 (E*d_ff x d), b2 (d).  pre and hidden (T x d_ff) are written
 * in expert-sorted row order (row i is token perm[i]) and kept for the
 * backward, like MoeDev (mod.rs:1416-1431). */
ASCA_API int asca_moe_fwd(const float* xn, const float* w1, const float* b1, const float* w2,
                          const float* b2, const int32_t* perm, const int32_t* offsets, int T, int d,
                          int d_ff, int n_experts, float* out, float* pre, float* hidden, void* stream);

/* HashMoE backward from dout (T x d): dW2 = hidden^T dout, db2 = colsum(dout),
 * dpre = dout w2_e^T * silu'(pre), db1 = colsum(dpre), dW1 = xn^T dpre,
 * dxn = dpre w1_e^T, per expert (Gpu::moe_bwd_dev, mod.rs:745-824; CPU
 * semantics HashMoe::backward, model.rs:339-497, before its RMSNorm backward).
 * With accumulate != 0 the weight and bias gradients are added to dw1, db1,
 * dw2, db2 (Param::grad accumulation); dxn is overwritten.  dpre_ws: T*d_ff
 * floats of workspace. */
ASCA_API int asca_moe_bwd(const float* xn, const float* w1, const float* w2, const float* pre,
                          const float* hidden, const int32_t* perm, const int32_t* offsets,
                          const float* dout, int T, int d, int d_ff, int n_experts, float* dxn,
                          float* dw1, float* db1, float* dw2, float* db2, float* dpre_ws, int accumulate,
                          void* stream);

/* ------------------------------------------- delta rule (chunked form) -- */

/* The chunked (WY/UT-transform) form of the same recurrence, specified but not
 * implemented by the reference (docs/SPEC_V2.md:50-69): chunks of C steps,
 * per chunk T = (I + strict_tril(diag(beta)(Gamma o K K^T)))^-1,
 * U = T diag(beta)(V - diag(gamma) K S), O = diag(gamma) Q S + tril(Gamma o Q K^T) U,
 * S' = gamma_C S + (diag(Gamma[C-1,:]) K)^T U, with every product on the
 * matrix cores (f32 MFMA) and the state carried across chunks by one d x d
 * product per chunk.  At C = 64, dh = 128 each direction is one fused
 * per-chunk kernel around a persistent state scan; other shapes run batched
 * GEMMs over chunks.  Same results as asca_delta_fwd /
 * asca_delta_bwd_raw (DeltaBlock::scan_cpu / bptt_cpu, rust/src/delta.rs:244-334,
 * 475-587) up to f32 rounding.
 *   q, k, v, d_o : (B*T, H*dh) bf16 (raw 16-bit patterns); alpha, beta : (B*T, H) f32
 *   o, dq, dk, dv : (B*T, H*dh) f32; dalpha, dbeta : (B*T, H) f32 (raw, not logits)
 *   1 <= C <= 64; dh a multiple of 4, at most 256.
 *   ws : asca_chunk_ws_bytes bytes; the forward leaves in it what the backward
 *   needs: call asca_chunk_bwd with the forward's ws and the same q, k, v (the
 *   backward reads the bf16 inputs, as the reference's backward keeps q, k, v
 *   resident in DeltaDev, rust/src/cuda/mod.rs:1386-1397). */
ASCA_API int asca_chunk_ws_bytes(int B, int T, int H, int dh, int C, size_t* bytes);
ASCA_API int asca_chunk_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* alpha,
                            const float* beta, float* o, void* ws, int B, int T, int H, int dh, int C,
                            void* stream);
ASCA_API int asca_chunk_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* d_o, void* ws,
                            float* dq, float* dk, float* dv, float* dalpha, float* dbeta, int B, int T, int H,
                            int dh, int C, void* stream);
/* The same chunked form on f32 q, k, v, d_o (any alignment), for the f32
 * recurrent configs (configs[1]: B32 T512 H8 dh64): the same math and outputs
 * as asca_chunk_fwd / asca_chunk_bwd, every per-chunk product a batched f32
 * MFMA GEMM over chunks at any C (1..64) and dh.  ws : asca_chunk_ws_bytes_f32
 * bytes (it holds unit-major f32 copies of q, k, v, so the backward takes only
 * d_o).  No reference counterpart: the reference's SPEC_V2 names the form
 * (docs/SPEC_V2.md:50-69) and its f32 path is the recurrence; these let the
 * MFMA route be measured against the recurrent kernels on the same f32
 * inputs. */
ASCA_API int asca_chunk_ws_bytes_f32(int B, int T, int H, int dh, int C, size_t* bytes);
ASCA_API int asca_chunk_fwd_f32(const float* q, const float* k, const float* v, const float* alpha,
                                const float* beta, float* o, void* ws, int B, int T, int H, int dh, int C,
                                void* stream);
ASCA_API int asca_chunk_bwd_f32(const float* d_o, void* ws, float* dq, float* dk, float* dv, float* dalpha,
                                float* dbeta, int B, int T, int H, int dh, int C, void* stream);

/* ----------------------------------------------------- training step -- */

/* A device-resident ASCA model (rust/src/model.rs:528-802): parameters,
 * gradients and AdamW moments in four flat f32 device buffers, tensors in the
 * reference's params() order -- embed (V x d), head (d x V), then per layer
 * delta.w_qkv (d x 3d), delta.b_qkv, delta.w_gate (d x 2H), delta.b_gate,
 * delta.w_o (d x d), delta.b_o, moe.w1 (d x E*d_ff), moe.b1, moe.w2
 * (E*d_ff x d), moe.b2 -- each starting at a 16-byte aligned offset
 * (asca_model_tensor_info).  It replaces the Rust host's Model + Param
 * residency of the reference's GPU backend (Param values/grads shuttled per
 * op, rust/src/cuda/mod.rs) by whole-step residency.  Parameters start at zero;
 * the caller uploads its initialisation into the params buffer. */
typedef struct asca_model asca_model;

ASCA_API int asca_model_create(int vocab, int d_model, int n_heads, int n_layers, int n_experts, int d_ff,
                               asca_model** out);
ASCA_API int asca_model_destroy(asca_model* model);
ASCA_API int asca_model_num_tensors(const asca_model* model, int* n);
ASCA_API int asca_model_tensor_info(const asca_model* model, int i, char* name, int name_len, size_t* offset,
                                   int* rows, int* cols);
/* Device pointers of the flat buffers (n_floats entries each). */
ASCA_API int asca_model_buffers(asca_model* model, size_t* n_floats, float** params, float** grads, float** m,
                                float** v);
/* AdamW hyper-parameters and step counter (AdamW::new / ::update,
 * rust/src/tensor.rs:381-402); the counter advances once per tensor per step. */
ASCA_API int asca_model_set_adamw(asca_model* model, float lr, float beta1, float beta2, float eps, float wd,
                                  uint32_t step);
ASCA_API int asca_model_adamw_step_count(const asca_model* model, uint32_t* step);

/* Model::forward + Model::backward after zero_grads (rust/src/train.rs:176-186):
 * ids, targets are device u32 arrays of batch*seq tokens (sequence b is rows
 * b*seq..); gradients are written into the grads buffer; *loss (device, may
 * be NULL) receives the mean cross-entropy.  The weight gradients run on a
 * second stream owned by the model (default priority, non-blocking), which
 * `stream` waits for before the call's last work: anything queued on `stream`
 * afterwards (or a synchronisation of it) sees every gradient. */
ASCA_API int asca_model_forward_backward(asca_model* model, const uint32_t* ids, const uint32_t* targets,
                                         int batch, int seq, float* loss, void* stream);
/* The optimiser step over every tensor (model.rs:797-802 / AdamW::update). */
ASCA_API int asca_model_adamw(asca_model* model, void* stream);
/* forward_backward followed by asca_model_adamw: one training step.  The
 * updates run on a third stream of the model, each group of tensors as soon as
 * its gradients are final (bit-identical to one update after the backward);
 * they are queued only after every launch of the backward was queued.  A
 * failure before the updates leaves parameters, moments and the step count
 * untouched (repeat the step); ASCA_ERR_PARTIAL_UPDATE means an update launch
 * failed after others were queued: some tensors moved by one step, the step
 * count did not (restore from a checkpoint).  Either way `stream` waits for
 * everything the call queued on the model's streams. */
ASCA_API int asca_model_train_step(asca_model* model, const uint32_t* ids, const uint32_t* targets, int batch,
                                   int seq, float* loss, void* stream);

/* Model::step for n_seq sequences at once, one token each (rust/src/model.rs:
 * 631-649; DeltaBlock::step delta.rs:341-411, HashMoe::step model.rs:308-337):
 * ids[s] (device u32) goes through the embedding, every layer's delta step on
 * the carried states and hashed-expert MoE, the final RMSNorm and the head.
 * The reference decodes on the CPU only, one sequence at a time.
 *   states : device f32, n_seq * asca_model_decode_state_floats() floats,
 *            layout (L, n_seq, H, dh, dh) row-major S[a][i] (zero for a new
 *            sequence), updated in place
 *   logits : device f32 (n_seq, V) */
ASCA_API int asca_model_decode_state_floats(const asca_model* model, size_t* per_seq);
ASCA_API int asca_model_decode_step(asca_model* model, const uint32_t* ids, int n_seq, float* states,
                                   float* logits, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* ASCA_HIP_H */
