// f32 GEMM on the CDNA4 matrix cores (v_mfma_f32_16x16x4_f32), with the
// operand/epilogue variants the model needs:
//
//   C = alpha * op(A) op(B) (+ bias per column) (+ beta * C)
//
// where op(A) is A (M x K, row-major) or A^T (A stored K x M), op(B) is B
// (K x N) or B^T (B stored N x K) -- the reference's matmul_f32 / matmul_ta_f32
// / matmul_ld_f32 family (rust/kernels/asca.cu:14-141) and Mat::matmul /
// matmul_ta / matmul_t (rust/src/tensor.rs:91-201).  On top of that:
//   - storage-row indirection per operand (row gather) and on C (row scatter),
//     replacing gather_rows_f32 / scatter_rows_f32 round trips (asca.cu:576-594);
//   - grouped launches over expert buckets (CSR offsets on the device): either
//     M varies per group (expert forward GEMMs, dpre, dxn) or K varies per
//     group (expert weight gradients), one launch for all experts;
//   - fused epilogues: bias + SiLU writing both pre and hidden (HashMoe
//     forward, rust/src/model.rs:236-248), and the SiLU backward
//     dpre = acc * s (1 + pre (1 - s)) (model.rs:432-440);
//   - split-K with f32 partials and a deterministic reduction, for the
//     K = tokens weight-gradient products that have few output tiles.
//
// Tiling: 256 threads, a 128 x 128 block tile, k-tiles of 32 double-buffered
// in LDS, four waves of 64 x 64.  Each operand keeps its global layout in LDS
// (no transposing stores): a k-contiguous tile is [mn][k] with a 36-float row
// stride, an mn-contiguous tile is [k][mn].  The MFMA k index is permuted
// inside every 16-k group (step s, lane l uses k = 4 (l / 16) + s) so every
// fragment read is one 16-byte ds_read: a [mn][k] read yields four k-steps of
// one 16-row tile, a [k][mn] read yields one k-step of four tiles whose rows
// are interleaved by 4.  The epilogue maps rows/columns back accordingly.
// Plain products whose grid fills whole rounds of the CUs, and the grouped-K
// expert weight gradients, take a 128 x 256 variant on 8 waves whose operand
// tiles go from global memory straight into LDS (described at dma_mainloop).
#include <mutex>
#include <type_traits>

#include "common.h"
#include "gemm.h"
#include "runtime.h"

namespace asca {

// Block tiles are (64 WM) x (64 WN) with one 64 x 64 wave tile per wave:
// 128 x 128 on 4 waves for the large products, 64 x 128 on 2 waves for the
// 64-row batched per-chunk products of the chunked delta rule.
constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 32;
constexpr int GM_LDK = GM_BK + 4;  // [mn][k] tile row stride (floats)

// floats of one LDS operand tile with R mn-rows
template <bool KC, int R>
constexpr int tile_floats() { return KC ? R * GM_LDK : GM_BK * R; }

ASCA_DEV float silu_ref(float x) { return x / (1.0f + expf(-x)); }

// 4 consecutive floats from p, of which n (<= 0 .. >= 4) are valid; the rest 0.
template <bool VEC>
ASCA_DEV float4 ld4(const float* p, int n) {
    if (VEC && n >= 4) return *reinterpret_cast<const float4*>(p);
    float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
    if (n > 0) r.x = p[0];
    if (n > 1) r.y = p[1];
    if (n > 2) r.z = p[2];
    if (n > 3) r.w = p[3];
    return r;
}

ASCA_DEV long srow(const int* rows, long off, long i) { return rows ? (long)rows[off + i] : off + i; }

// Global -> registers for one operand tile (8 R / NT float4 per thread).
//   KC (k-contiguous, stored [mn][k]): R mn-rows x 32 k, 8 threads per row.
//   MC (mn-contiguous, stored [k][mn]): 32 k-rows x R mn, R/4 threads per row.
// `lim_mn`, `lim_k`: valid extents relative to the tile origin.
template <bool KC, bool VEC, int R, int NT>
ASCA_DEV void tile_load(float4 (&r)[8 * R / NT], const float* base, long ld, const int* rows, long row_off,
                        int mn0, int lim_mn, long k0, long lim_k, int tid) {
#pragma unroll
    for (int j = 0; j < 8 * R / NT; ++j) {
        const int sl = tid + NT * j;
        if constexpr (KC) {
            const int rr = sl >> 3;
            const int kk = 4 * (sl & 7);
            const bool ok = rr < lim_mn;
            const long sr = ok ? srow(rows, row_off, mn0 + rr) : 0;
            r[j] = ld4<VEC>(base + sr * ld + k0 + kk, ok ? (int)min(lim_k - kk, 4L) : 0);
        } else {
            const int kr = sl / (R / 4);
            const int mm = 4 * (sl % (R / 4));
            const bool ok = kr < lim_k;
            const long sr = ok ? srow(rows, row_off, k0 + kr) : 0;
            r[j] = ld4<VEC>(base + sr * ld + mn0 + mm, ok ? min(lim_mn - mm, 4) : 0);
        }
    }
}

// Row offsets (source row * ld) of this thread's mn-rows of a k-contiguous
// tile; they do not change along K, so they are read once per block.
template <int R, int NT>
ASCA_DEV void tile_rows(long (&ro)[8 * R / NT], long ld, const int* rows, long row_off, int mn0, int lim_mn,
                        int tid) {
#pragma unroll
    for (int j = 0; j < 8 * R / NT; ++j) {
        const int rr = (tid + NT * j) >> 3;
        ro[j] = rr < lim_mn ? srow(rows, row_off, mn0 + rr) * ld : 0;
    }
}

// Row offsets (source row * ld) of this thread's k-rows of an mn-contiguous
// tile whose storage rows are gathered (rows != null): read one k-tile ahead
// of its loads, so no load waits on the index read before it.  Rows past the
// valid extent are clamped to the last valid one.
template <int R, int NT>
ASCA_DEV void tile_krows(long (&ro)[8 * R / NT], long ld, const int* rows, long row_off, long k0, long lim_k,
                         int tid) {
#pragma unroll
    for (int j = 0; j < 8 * R / NT; ++j) {
        const int kr = (tid + NT * j) / (R / 4);
        ro[j] = (long)rows[row_off + k0 + min((long)kr, lim_k - 1)] * ld;
    }
}

// As tile_load for a tile that lies wholly inside the operand (aligned, no
// edge): unconditional 16-byte loads; a k-contiguous tile takes its row
// offsets from tile_rows, a gathered mn-contiguous one from tile_krows.
template <bool KC, int R, int NT>
ASCA_DEV void tile_load_full(float4 (&r)[8 * R / NT], const float* base, long ld, const int* rows, long row_off,
                             const long (&ro)[8 * R / NT], int mn0, long k0, int tid) {
#pragma unroll
    for (int j = 0; j < 8 * R / NT; ++j) {
        const int sl = tid + NT * j;
        if constexpr (KC) {
            const int kk = 4 * (sl & 7);
            r[j] = *reinterpret_cast<const float4*>(base + ro[j] + k0 + kk);
        } else {
            const int kr = sl / (R / 4), mm = 4 * (sl % (R / 4));
            const long off = rows ? ro[j] : (row_off + k0 + kr) * ld;
            r[j] = *reinterpret_cast<const float4*>(base + off + mn0 + mm);
        }
    }
}

template <bool KC, int R, int NT>
ASCA_DEV void tile_store(const float4 (&r)[8 * R / NT], float* t, int tid) {
#pragma unroll
    for (int j = 0; j < 8 * R / NT; ++j) {
        const int sl = tid + NT * j;
        if constexpr (KC)
            *reinterpret_cast<float4*>(t + (sl >> 3) * GM_LDK + 4 * (sl & 7)) = r[j];
        else
            *reinterpret_cast<float4*>(t + (sl / (R / 4)) * R + 4 * (sl % (R / 4))) = r[j];
    }
}

// Fragments of one 16-k group h for the wave's 64 mn-rows starting at w0:
// f[s][t] = operand value of MFMA k-step s for 16-row tile t.
template <bool KC, int R>
ASCA_DEV void frag_read(float (&f)[4][4], const float* t, int w0, int h, int lane) {
    if constexpr (KC) {
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            const float4 v =
                *reinterpret_cast<const float4*>(t + (w0 + 16 * x + (lane & 15)) * GM_LDK + 16 * h + 4 * (lane >> 4));
            f[0][x] = v.x;
            f[1][x] = v.y;
            f[2][x] = v.z;
            f[3][x] = v.w;
        }
    } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float4 v =
                *reinterpret_cast<const float4*>(t + (16 * h + 4 * (lane >> 4) + s) * R + w0 + 4 * (lane & 15));
            f[s][0] = v.x;
            f[s][1] = v.y;
            f[s][2] = v.z;
            f[s][3] = v.w;
        }
    }
}

// As frag_read for NTL 16-row tiles (NTL = 2 or 4): the wave's 16 NTL
// mn-rows starting at w0.  In the mn-contiguous layout tile x holds the rows
// w0 + NTL i + x (i = lane % 16), one 8- or 16-byte read per k-step.
template <bool KC, int R, int NTL>
ASCA_DEV void frag_read_n(float (&f)[4][NTL], const float* t, int w0, int h, int lane) {
    if constexpr (NTL == 4) {
        frag_read<KC, R>(f, t, w0, h, lane);
    } else if constexpr (KC) {
#pragma unroll
        for (int x = 0; x < NTL; ++x) {
            const float4 v =
                *reinterpret_cast<const float4*>(t + (w0 + 16 * x + (lane & 15)) * GM_LDK + 16 * h + 4 * (lane >> 4));
            f[0][x] = v.x;
            f[1][x] = v.y;
            f[2][x] = v.z;
            f[3][x] = v.w;
        }
    } else {
        static_assert(NTL == 2, "tile count");
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float2 v =
                *reinterpret_cast<const float2*>(t + (16 * h + 4 * (lane >> 4) + s) * R + w0 + 2 * (lane & 15));
            f[s][0] = v.x;
            f[s][1] = v.y;
        }
    }
}

// acc (4 x TN tiles of 16 x 16) += the 16-k group whose fragments are fa, fb.
template <int TN>
ASCA_DEV void mfma_4xn(f32x4 (&acc)[4][TN], const float (&fa)[4][4], const float (&fb)[4][TN]) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int y = 0; y < TN; ++y)
                acc[x][y] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[s][x], fb[s][y], acc[x][y], 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Direct-to-LDS main loop (128 x 256 block tile, 8 waves of 64 x 64).
//
// The operand tiles go from global memory straight into LDS with
// global_load_lds_dwordx4 (no register staging, no ds_write): each instruction
// writes 64 lanes x 16 bytes contiguously at M0, and the lane -> global address
// map is free, so every 1 KB chunk of a stage is laid out exactly as the MFMA
// fragment reads want it: lane l reads the 16 bytes at chunk + 16 l (linear,
// no bank conflict, no padding).  A stage is one k-tile of 16:
//   k-contiguous operand ([mn][k] in memory): chunk c holds mn = 16 c + l % 16,
//     k = 4 (l / 16) .. +3, i.e. the four k-steps of one 16-row tile;
//   mn-contiguous operand ([k][mn]): chunk c holds k = 4 (l / 16) + c % 4,
//     mn = 64 (c / 4) + 4 (l % 16) .. +3, i.e. one k-step of four tiles whose
//     rows are interleaved by 4 (the same fragment semantics as the register
//     path, so the epilogue is shared).
// A (128 mn) has 8 chunks, B (256 mn) 16: wave w loads A chunk w and B chunks
// 2w, 2w+1.  Three stages: step t waits for its own loads of tile t+1, passes
// a barrier (every wave's part landed, every wave done reading tile t-1),
// issues tile t+2 into the stage of tile t-1, reads the fragments of tile t+1
// and multiplies tile t from registers.  Lanes whose k lies past the K range
// load from a zero block instead (k tails, grouped K); rows past M or N are
// clamped into the tile (their results are never stored).
//
// The loads are written as inline assembly: the compiler's own tracking of
// LDS DMA makes every LDS read wait for all outstanding loads.  The loop waits
// for them itself (s_waitcnt vmcnt(0) before each barrier), and waits for all
// of them before the kernel ends, so no load lands in LDS after the block.
constexpr int DMA_STAGES = 3, DMA_BK = 16;
// bytes of one stage: 8 chunks of A (128 rows) and 4 WN of B (64 WN columns)
template <int WN>
constexpr int dma_stage_bytes() { return (8 + 4 * WN) * 1024; }

__device__ float4 g_dma_zero = {0.f, 0.f, 0.f, 0.f};  // read-only source for k past the range

ASCA_DEV void dma16(const float* g, unsigned lds_byte) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_byte), "v"(g) : "memory", "m0");
}
ASCA_DEV void dma_wait_all() { __builtin_amdgcn_s_waitcnt(0xF70); }  // vmcnt(0)

// One lane's share of one chunk of an operand: source of the next k-tile.
struct DmaSrc {
    const float* p;  // k-contiguous, or mn-contiguous without row gather: source at the next k-tile
    long step;       // advance per k-tile (floats)
    long col;        // mn-contiguous: column of the lane's float4
    int kofs;        // the lane's k within a k-tile
    int idx;         // mn-contiguous with row gather: storage row of the next k-tile
};

template <bool KC>
ASCA_DEV DmaSrc dma_src(int c, int lane, const float* base, long ld, const int* rows, long row_off, int mn0,
                        int lim_mn, long K_lo, long K_hi) {
    DmaSrc d;
    if constexpr (KC) {
        int mn = 16 * c + (lane & 15);
        if (mn >= lim_mn) mn = 0;
        d.kofs = 4 * (lane >> 4);
        d.p = base + srow(rows, row_off, mn0 + mn) * ld + K_lo + d.kofs;
        d.step = DMA_BK;
        d.col = 0;
        d.idx = 0;
    } else {
        d.kofs = 4 * (lane >> 4) + (c & 3);
        const int mm = min(64 * (c >> 2) + 4 * (lane & 15), lim_mn - 4);
        d.col = mn0 + mm;
        d.p = base + (row_off + K_lo + d.kofs) * ld + d.col;
        d.step = (long)DMA_BK * ld;
        d.idx = rows ? rows[row_off + min(K_lo + d.kofs, K_hi - 1)] : 0;
    }
    return d;
}

// Issue k-tile t of one chunk into LDS byte address `dst`, then advance.  In
// a k-tile that reaches past K_hi (`tail`, the last one at most) a lane whose
// k is past K_hi reads the zero block.
template <bool KC>
ASCA_DEV void dma_issue(DmaSrc& d, long t, const float* base, long ld, const int* rows, long row_off, long K_lo,
                        long K_hi, bool tail, unsigned dst) {
    const long k = K_lo + t * DMA_BK + d.kofs;
    const float* src = d.p;
    if constexpr (!KC) {
        if (rows) {  // uniform
            src = base + (long)d.idx * ld + d.col;
            d.idx = rows[row_off + min(k + DMA_BK, K_hi - 1)];  // next k-tile's storage row
        }
    }
    if (tail && k >= K_hi) src = reinterpret_cast<const float*>(&g_dma_zero);  // tail: uniform
    d.p += d.step;
    dma16(src, dst);
}

template <bool TA, bool TB, int WN>
ASCA_DEV void dma_mainloop(f32x4 (&acc)[4][4], const float* A, const float* B, const GemmArgs& p, long a_off,
                           long b_off, int m0, int n0, int lim_m, int lim_n, long K_lo, long K_hi, int w, int lane,
                           int wm, int wn) {
    constexpr bool A_KC = !TA, B_KC = TB;
    constexpr int STAGE_B = dma_stage_bytes<WN>();
    constexpr int APW = 4 / WN;  // A chunks per wave (8 chunks over 2 WN waves); B chunks: 2 per wave
    extern __shared__ float4 lds4[];
    const float4* lds = lds4;
    const unsigned lds_b = (unsigned)(unsigned long)((__attribute__((address_space(3))) float4*)lds4);
    const int wu = __builtin_amdgcn_readfirstlane(w);
    DmaSrc sa[APW];
#pragma unroll
    for (int j = 0; j < APW; ++j)
        sa[j] = dma_src<A_KC>(APW * wu + j, lane, A, p.lda, p.a_rows, a_off, m0, lim_m, K_lo, K_hi);
    DmaSrc sb0 = dma_src<B_KC>(2 * wu, lane, B, p.ldb, p.b_rows, b_off, n0, lim_n, K_lo, K_hi);
    DmaSrc sb1 = dma_src<B_KC>(2 * wu + 1, lane, B, p.ldb, p.b_rows, b_off, n0, lim_n, K_lo, K_hi);
    const unsigned ca = lds_b + (unsigned)(APW * wu) * 1024u, cb = lds_b + (unsigned)(8 + 2 * wu) * 1024u;
    // tile t into stage S (compile-time)
    const long t_tail = (K_hi - K_lo) / DMA_BK;  // first k-tile not wholly inside the K range
    // TL (compile-time): tile t may reach past K_hi (only then are the lanes'
    // k checked against it)
    auto issue = [&](long t, auto S, auto TL) {
        constexpr unsigned so = (unsigned)decltype(S)::value * STAGE_B;
        const bool tail = decltype(TL)::value && t >= t_tail;
#pragma unroll
        for (int j = 0; j < APW; ++j)
            dma_issue<A_KC>(sa[j], t, A, p.lda, p.a_rows, a_off, K_lo, K_hi, tail, ca + 1024u * j + so);
        dma_issue<B_KC>(sb0, t, B, p.ldb, p.b_rows, b_off, K_lo, K_hi, tail, cb + so);
        dma_issue<B_KC>(sb1, t, B, p.ldb, p.b_rows, b_off, K_lo, K_hi, tail, cb + 1024u + so);
    };
    float fa[2][4][4], fb[2][4][4];
    // fragments of stage S into buffer BUF (both compile-time): 16-byte reads
    // at chunk + 16 lane
    const float4* rb = lds + lane;
    const int ax = A_KC ? (wm >> 4) : (wm >> 6) * 4, bx = 8 + (B_KC ? (wn >> 4) : (wn >> 6) * 4);
    auto rd = [&](auto S, auto BUF) {
        constexpr int st = decltype(S)::value * (STAGE_B / 16), buf = decltype(BUF)::value;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = rb[st + (ax + i) * 64];
            if constexpr (A_KC) {
                fa[buf][0][i] = v.x; fa[buf][1][i] = v.y; fa[buf][2][i] = v.z; fa[buf][3][i] = v.w;
            } else {
                fa[buf][i][0] = v.x; fa[buf][i][1] = v.y; fa[buf][i][2] = v.z; fa[buf][i][3] = v.w;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = rb[st + (bx + i) * 64];
            if constexpr (B_KC) {
                fb[buf][0][i] = v.x; fb[buf][1][i] = v.y; fb[buf][2][i] = v.z; fb[buf][3][i] = v.w;
            } else {
                fb[buf][i][0] = v.x; fb[buf][i][1] = v.y; fb[buf][i][2] = v.z; fb[buf][i][3] = v.w;
            }
        }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    const long nk = (K_hi - K_lo + DMA_BK - 1) / DMA_BK;  // > 0
    using Tail = std::true_type;
    using NoTail = std::false_type;
    issue(0, I0{}, Tail{});
    if (nk > 1) issue(1, I1{}, Tail{});
    dma_wait_all();
    __syncthreads();
    rd(I0{}, I0{});
    // Step t at phase P = t % 6: tile t in buffer P % 2 and stage P % 3.
    // The scheduling barriers keep the fragment reads for the next step ahead
    // of the products and the next step's wait and barrier behind them (left
    // alone, the compiler moved the reads down to the barrier, whose wait then
    // fell on them).
    auto step = [&](long t, auto P, auto TL) {
        constexpr int ph = decltype(P)::value;
        dma_wait_all();
        __syncthreads();
        if (t + 2 < nk) issue(t + 2, std::integral_constant<int, (ph + 2) % 3>{}, TL);
        rd(std::integral_constant<int, (ph + 1) % 3>{}, std::integral_constant<int, (ph + 1) % 2>{});
        __builtin_amdgcn_sched_barrier(0);
        mfma_4xn<4>(acc, fa[ph % 2], fb[ph % 2]);
        __builtin_amdgcn_sched_barrier(0);
    };
    using P3 = std::integral_constant<int, 3>;
    using P4 = std::integral_constant<int, 4>;
    using P5 = std::integral_constant<int, 5>;
    long t = 0;
    // steps whose issued tile t + 2 lies wholly inside the K range (t + 2 < t_tail)
    for (; t + 6 < nk && t + 7 < t_tail; t += 6) {
        step(t, I0{}, NoTail{});
        step(t + 1, I1{}, NoTail{});
        step(t + 2, I2{}, NoTail{});
        step(t + 3, P3{}, NoTail{});
        step(t + 4, P4{}, NoTail{});
        step(t + 5, P5{}, NoTail{});
    }
    for (; t + 6 < nk; t += 6) {
        step(t, I0{}, Tail{});
        step(t + 1, I1{}, Tail{});
        step(t + 2, I2{}, Tail{});
        step(t + 3, P3{}, Tail{});
        step(t + 4, P4{}, Tail{});
        step(t + 5, P5{}, Tail{});
    }
    // the last 1..6 steps (the fragments read past the last tile are unused)
    do {
        step(t, I0{}, Tail{});
        if (t + 1 >= nk) break;
        step(t + 1, I1{}, Tail{});
        if (t + 2 >= nk) break;
        step(t + 2, I2{}, Tail{});
        if (t + 3 >= nk) break;
        step(t + 3, P3{}, Tail{});
        if (t + 4 >= nk) break;
        step(t + 4, P4{}, Tail{});
        if (t + 5 >= nk) break;
        step(t + 5, P5{}, Tail{});
    } while (false);
    dma_wait_all();
}

// Block tile (64 WM) x (16 TNW WN) on WM x WN waves; a wave owns 64 rows x
// 16 TNW columns (TNW = 4, or 2 for the narrower tile that lets three blocks
// share a CU).
template <bool TA, bool TB, int EPI, bool VEC, int WM, int WN, int TNW = 4, bool DMA = false>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(WM * WN >= 4 ? 2 : 1))) void gemm_k(GemmArgs p) {
    constexpr int NT = 64 * WM * WN, BM = 64 * WM, BN = 16 * TNW * WN;
    constexpr bool A_KC = !TA, B_KC = TB;
    constexpr int A_F = tile_floats<A_KC, BM>();
    constexpr int B_F = tile_floats<B_KC, BN>();
    extern __shared__ float4 lds4[];
    float* lds = reinterpret_cast<float*>(lds4);

    // block -> tile, XCD-aware: hardware places block i on XCD i % 8, so give
    // each XCD a contiguous run of logical tiles (neighbours share operand rows)
    int L = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) L = (L & 7) * (nb >> 3) + (L >> 3);
    int g = 0, tm, tn = L % p.tiles_n;
    int Mg = p.M;
    long K_lo = 0, K_hi = p.K, goff_g = 0;
    if (p.gmode == 1) {
        int mt = L / p.tiles_n;
        for (; g < p.ngroups; ++g) {
            const int a = p.goff[g], b = p.goff[g + 1];
            const int nt = (b - a + BM - 1) / BM;
            if (mt < nt) break;
            mt -= nt;
        }
        if (g >= p.ngroups) return;  // surplus block (grid is an upper bound)
        tm = mt;
        goff_g = p.goff[g];
        Mg = p.goff[g + 1] - p.goff[g];
    } else if (p.gmode == 2) {
        const int r = L / p.tiles_n;
        tm = r % p.tiles_m;
        g = r / p.tiles_m;
        goff_g = p.goff[g];
        K_hi = p.goff[g + 1] - p.goff[g];
    } else if (p.gmode == 3) {
        const int r = L / p.tiles_n;
        tm = r % p.tiles_m;
        g = r / p.tiles_m;
    } else {
        tm = L / p.tiles_n;
        K_lo = (long)blockIdx.y * p.k_per_split;
        K_hi = min((long)p.K, K_lo + p.k_per_split);
    }
    const int m0 = tm * BM, n0 = tn * BN;
    const float* A = p.A + g * p.a_gs;
    const float* B = p.B + g * p.b_gs;
    float* C = p.C + g * p.c_gs + (long)blockIdx.y * p.c_split_stride;
    const float* bias = p.bias ? p.bias + g * p.bias_gs : nullptr;
    const float* resid = p.resid ? p.resid + g * p.r_gs : nullptr;
    const long a_off = ((p.gmode == 1 && !TA) || (p.gmode == 2 && TA)) ? goff_g : 0;
    const long b_off = (p.gmode == 2 && !TB) ? goff_g : 0;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = (w / WN) * 64, wn = (w % WN) * 16 * TNW;
    const int lim_m = Mg - m0, lim_n = p.N - n0;

    f32x4 acc[4][TNW];
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < TNW; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};

    if constexpr (DMA) {
        static_assert(WM == 2 && (WN == 4 || WN == 2) && TNW == 4 && VEC, "direct-to-LDS tile");
        if (K_hi > K_lo)
            dma_mainloop<TA, TB, WN>(acc, A, B, p, a_off, b_off, m0, n0, lim_m, lim_n, K_lo, K_hi, w, lane, wm, wn);
    } else {
    const long nk = (K_hi - K_lo + GM_BK - 1) / GM_BK;
    float4 ra[8 * BM / NT], rb[8 * BN / NT];
    // interior blocks (whole tiles in M and N) load without edge checks,
    // except in a partial last k-tile
    const bool interior = VEC && lim_m >= BM && lim_n >= BN;
    long roa[8 * BM / NT], rob[8 * BN / NT];
    if (A_KC) tile_rows<BM, NT>(roa, p.lda, p.a_rows, a_off, m0, lim_m, tid);
    if (B_KC) tile_rows<BN, NT>(rob, p.ldb, p.b_rows, b_off, n0, lim_n, tid);
    // gathered mn-contiguous operands: the row offsets of k-tile kt
    auto krows = [&](long kt) {
        const long k0 = K_lo + min(kt, nk - 1) * GM_BK;
        if (!A_KC && p.a_rows) tile_krows<BM, NT>(roa, p.lda, p.a_rows, a_off, k0, K_hi - k0, tid);
        if (!B_KC && p.b_rows) tile_krows<BN, NT>(rob, p.ldb, p.b_rows, b_off, k0, K_hi - k0, tid);
    };
    auto load = [&](long k0) {
        if (interior && K_hi - k0 >= GM_BK) {
            tile_load_full<A_KC, BM, NT>(ra, A, p.lda, p.a_rows, a_off, roa, m0, k0, tid);
            tile_load_full<B_KC, BN, NT>(rb, B, p.ldb, p.b_rows, b_off, rob, n0, k0, tid);
        } else {
            tile_load<A_KC, VEC, BM, NT>(ra, A, p.lda, p.a_rows, a_off, m0, lim_m, k0, K_hi - k0, tid);
            tile_load<B_KC, VEC, BN, NT>(rb, B, p.ldb, p.b_rows, b_off, n0, lim_n, k0, K_hi - k0, tid);
        }
    };
    // Two halves per k-tile kt, split by one barrier.  Each half multiplies
    // fragments that are already in registers while the other half's
    // fragments are read:
    //   A(kt): MFMAs of 16-k group 0 of kt | read group 1 of kt; store the
    //          registers holding k-tile kt+1 to the other LDS buffer
    //   B(kt): MFMAs of group 1 of kt | read group 0 of kt+1; issue the
    //          global loads of k-tile kt+2 into the registers
    // so a global load has a whole half plus most of the next to arrive.  The
    // buffer written in A(kt) was last read in A(kt-1), before the barrier of
    // kt-1.  Near the end the k-tile loaded is clamped to the last one (a
    // repeated load that is never stored).
    float fa0[4][4], fb0[4][TNW], fa1[4][4], fb1[4][TNW];
    if (nk > 0) {
        krows(0);
        load(K_lo);
        krows(1);
        tile_store<A_KC, BM, NT>(ra, lds, tid);
        tile_store<B_KC, BN, NT>(rb, lds + A_F, tid);
        load(K_lo + (nk > 1 ? GM_BK : 0));
        krows(2);
        __syncthreads();
        frag_read<A_KC, BM>(fa0, lds, wm, 0, lane);
        frag_read_n<B_KC, BN, TNW>(fb0, lds + A_F, wn, 0, lane);
        for (long kt = 0; kt < nk - 1; ++kt) {
            float* const Cs = lds + (kt & 1) * (A_F + B_F);
            float* const Ns = lds + ((kt + 1) & 1) * (A_F + B_F);
            frag_read<A_KC, BM>(fa1, Cs, wm, 1, lane);
            frag_read_n<B_KC, BN, TNW>(fb1, Cs + A_F, wn, 1, lane);
            mfma_4xn<TNW>(acc, fa0, fb0);
            tile_store<A_KC, BM, NT>(ra, Ns, tid);
            tile_store<B_KC, BN, NT>(rb, Ns + A_F, tid);
            __syncthreads();
            frag_read<A_KC, BM>(fa0, Ns, wm, 0, lane);
            frag_read_n<B_KC, BN, TNW>(fb0, Ns + A_F, wn, 0, lane);
            load(K_lo + min(kt + 2, nk - 1) * GM_BK);
            krows(kt + 3);
            mfma_4xn<TNW>(acc, fa1, fb1);
        }
        float* const Ls = lds + ((nk - 1) & 1) * (A_F + B_F);
        frag_read<A_KC, BM>(fa1, Ls, wm, 1, lane);
        frag_read_n<B_KC, BN, TNW>(fb1, Ls + A_F, wn, 1, lane);
        mfma_4xn<TNW>(acc, fa0, fb0);
        mfma_4xn<TNW>(acc, fa1, fb1);
    }
    }

    // epilogue: result register r of tile (x, y) sits at tile row 4 (lane / 16) + r,
    // tile column lane % 16.  Element y of a lane's row is column nc0 + NS y.
    // Every load the epilogue needs is unconditional (indices clamped into the
    // operand) and issued ahead of its use: the bias once per thread, the scatter
    // indices, residual, C and pre of four rows at a time.  A load under a
    // per-element condition is waited for on its own, one latency per element.
    constexpr int NS = B_KC ? 16 : 1;
    const int nc0 = B_KC ? n0 + wn + (lane & 15) : n0 + wn + TNW * (lane & 15);
    const int nmax = p.N - 1;
    float bv[TNW];
    if (bias) {
#pragma unroll
        for (int y = 0; y < TNW; ++y) bv[y] = bias[min(nc0 + NS * y, nmax)];
    }
    const bool add_c = EPI == EPI_STORE && p.beta != 0.0f;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
        long srt[4], crow[4];
        bool rok[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tr = 4 * (lane >> 4) + r;
            const int m = m0 + wm + (A_KC ? 16 * x + tr : 4 * tr + x);
            rok[r] = m < Mg;
            srt[r] = (p.gmode == 1 ? goff_g : 0) + min(m, Mg - 1);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) crow[r] = p.c_rows ? (long)p.c_rows[srt[r]] : srt[r];
        float lr[4][TNW], lc[4][TNW], la[4][TNW];
        if constexpr (EPI == EPI_STORE) {
            if (resid) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int y = 0; y < TNW; ++y) lr[r][y] = resid[crow[r] * p.ld_resid + min(nc0 + NS * y, nmax)];
            }
            if (add_c) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int y = 0; y < TNW; ++y) lc[r][y] = C[crow[r] * p.ldc + min(nc0 + NS * y, nmax)];
            }
        } else if constexpr (EPI == EPI_SILU_BWD) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int y = 0; y < TNW; ++y) la[r][y] = p.aux[srt[r] * p.ld_aux + min(nc0 + NS * y, nmax)];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (!rok[r]) continue;
            float* Cr = C + crow[r] * p.ldc;
            float o[TNW], hb[TNW];
#pragma unroll
            for (int y = 0; y < TNW; ++y) {
                float a = p.alpha * acc[x][y][r];
                if (bias) a += bv[y];
                if constexpr (EPI == EPI_STORE) {
                    if (add_c) a += p.beta * lc[r][y];
                    if (resid) a += lr[r][y];
                } else if constexpr (EPI == EPI_SILU) {
                    hb[y] = silu_ref(a);
                } else {
                    const float pr = la[r][y];
                    const float sg = 1.0f / (1.0f + expf(-pr));
                    a = acc[x][y][r] * (sg * (1.0f + pr * (1.0f - sg)));
                }
                o[y] = a;
            }
            if constexpr (!B_KC) {
                // columns nc0 .. nc0 + TNW - 1 of one row
                if (nc0 >= p.N) continue;
                const int cnt = min(p.N - nc0, TNW);
                const long ao = srt[r] * p.ld_aux + nc0;
                if (VEC && cnt == TNW && TNW == 4) {
                    *reinterpret_cast<float4*>(Cr + nc0) = make_float4(o[0], o[1], o[TNW - 2], o[TNW - 1]);
                    if constexpr (EPI == EPI_SILU)
                        *reinterpret_cast<float4*>(p.aux_out + ao) =
                            make_float4(hb[0], hb[1], hb[TNW - 2], hb[TNW - 1]);
                } else if (VEC && cnt == TNW && TNW == 2) {
                    *reinterpret_cast<float2*>(Cr + nc0) = make_float2(o[0], o[TNW - 1]);
                    if constexpr (EPI == EPI_SILU)
                        *reinterpret_cast<float2*>(p.aux_out + ao) = make_float2(hb[0], hb[TNW - 1]);
                } else {
#pragma unroll
                    for (int y = 0; y < TNW; ++y)
                        if (y < cnt) {
                            Cr[nc0 + y] = o[y];
                            if constexpr (EPI == EPI_SILU) p.aux_out[ao + y] = hb[y];
                        }
                }
            } else {
#pragma unroll
                for (int y = 0; y < TNW; ++y) {
                    const int n = nc0 + 16 * y;
                    if (n >= p.N) continue;
                    Cr[n] = o[y];
                    if constexpr (EPI == EPI_SILU) p.aux_out[srt[r] * p.ld_aux + n] = hb[y];
                }
            }
        }
    }
}

// Persistent batched products (gmode 3, plain epilogue): a block walks work
// items (batch g, tile tm, tn) with a stride of gridDim.x and the k-tile
// pipeline runs across item boundaries, so the first k-tile of the next item
// loads while the last one of the current item is multiplied.  The per-chunk
// products of the chunked delta rule are small (K = 64 or 128), and as one
// block per product each paid its whole load latency up front.
template <bool TA, bool TB, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(1, 2))) void gemm_batched_k(
    GemmArgs p) {
    constexpr int NT = 64 * WM * WN, BM = 64 * WM, BN = 64 * WN;
    constexpr bool A_KC = !TA, B_KC = TB;
    constexpr int A_F = tile_floats<A_KC, BM>();
    constexpr int B_F = tile_floats<B_KC, BN>();
    extern __shared__ float4 lds4[];
    float* lds = reinterpret_cast<float*>(lds4);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = (w / WN) * 64, wn = (w % WN) * 64;
    const int per = p.tiles_m * p.tiles_n;
    const long items = (long)p.ngroups * per;
    const int nk = (p.K + GM_BK - 1) / GM_BK;  // the host guarantees K > 0
    long item = blockIdx.x;
    if (item >= items) return;

    long g = item / per;
    int m0 = (int)(item % per) / p.tiles_n * BM, n0 = (int)(item % per) % p.tiles_n * BN;
    const float* A = p.A + g * p.a_gs;
    const float* B = p.B + g * p.b_gs;
    float4 ra[8 * BM / NT], rb[8 * BN / NT];
    tile_load<A_KC, true, BM, NT>(ra, A, p.lda, nullptr, 0, m0, p.M - m0, 0, p.K, tid);
    tile_load<B_KC, true, BN, NT>(rb, B, p.ldb, nullptr, 0, n0, p.N - n0, 0, p.K, tid);
    tile_store<A_KC, BM, NT>(ra, lds, tid);
    tile_store<B_KC, BN, NT>(rb, lds + A_F, tid);
    __syncthreads();
    int it = 0;  // k-iterations so far (LDS buffer parity)
    for (;;) {
        const long next = item + gridDim.x;
        const bool has_next = next < items;
        const long gn = has_next ? next / per : g;
        const int rn = has_next ? (int)(next % per) : 0;
        const int m0n = rn / p.tiles_n * BM, n0n = rn % p.tiles_n * BN;
        const float* An = p.A + gn * p.a_gs;
        const float* Bn = p.B + gn * p.b_gs;
        f32x4 acc[4][4];
#pragma unroll
        for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int y = 0; y < 4; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int kt = 0; kt < nk; ++kt, ++it) {
            const float* As = lds + (it & 1) * (A_F + B_F);
            const float* Bs = As + A_F;
            const bool more = kt + 1 < nk || has_next;
            if (kt + 1 < nk) {
                const long k0 = (long)(kt + 1) * GM_BK;
                tile_load<A_KC, true, BM, NT>(ra, A, p.lda, nullptr, 0, m0, p.M - m0, k0, p.K - k0, tid);
                tile_load<B_KC, true, BN, NT>(rb, B, p.ldb, nullptr, 0, n0, p.N - n0, k0, p.K - k0, tid);
            } else if (has_next) {
                tile_load<A_KC, true, BM, NT>(ra, An, p.lda, nullptr, 0, m0n, p.M - m0n, 0, p.K, tid);
                tile_load<B_KC, true, BN, NT>(rb, Bn, p.ldb, nullptr, 0, n0n, p.N - n0n, 0, p.K, tid);
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float fa[4][4], fb[4][4];
                frag_read<A_KC, BM>(fa, As, wm, h, lane);
                frag_read<B_KC, BN>(fb, Bs, wn, h, lane);
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int x = 0; x < 4; ++x)
#pragma unroll
                        for (int y = 0; y < 4; ++y)
                            acc[x][y] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[s][x], fb[s][y], acc[x][y], 0, 0, 0);
            }
            if (more) {
                float* Ns = lds + ((it + 1) & 1) * (A_F + B_F);
                tile_store<A_KC, BM, NT>(ra, Ns, tid);
                tile_store<B_KC, BN, NT>(rb, Ns + A_F, tid);
            }
            __syncthreads();
        }
        // epilogue of this item: C = alpha acc + bias + beta C + resid
        float* C = p.C + g * p.c_gs;
        const float* bias = p.bias ? p.bias + g * p.bias_gs : nullptr;
        const float* resid = p.resid ? p.resid + g * p.r_gs : nullptr;
#pragma unroll
        for (int x = 0; x < 4; ++x) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tr = 4 * (lane >> 4) + r;
                const int m = m0 + wm + (A_KC ? 16 * x + tr : 4 * tr + x);
                if (m >= p.M) continue;
                float* Cr = C + (long)m * p.ldc;
                const float* Rr = resid ? resid + (long)m * p.ld_resid : nullptr;
                if constexpr (!B_KC) {
                    const int n = n0 + wn + 4 * (lane & 15);
                    if (n >= p.N) continue;
                    float o[4];
#pragma unroll
                    for (int y = 0; y < 4; ++y) {
                        float a = p.alpha * acc[x][y][r];
                        if (n + y < p.N) {
                            if (bias) a += bias[n + y];
                            if (p.beta != 0.0f) a += p.beta * Cr[n + y];
                            if (Rr) a += Rr[n + y];
                        }
                        o[y] = a;
                    }
                    if (n + 3 < p.N) {
                        *reinterpret_cast<float4*>(Cr + n) = make_float4(o[0], o[1], o[2], o[3]);
                    } else {
#pragma unroll
                        for (int y = 0; y < 4; ++y)
                            if (n + y < p.N) Cr[n + y] = o[y];
                    }
                } else {
#pragma unroll
                    for (int y = 0; y < 4; ++y) {
                        const int n = n0 + wn + 16 * y + (lane & 15);
                        if (n >= p.N) continue;
                        float a = p.alpha * acc[x][y][r];
                        if (bias) a += bias[n];
                        if (p.beta != 0.0f) a += p.beta * Cr[n];
                        if (Rr) a += Rr[n];
                        Cr[n] = a;
                    }
                }
            }
        }
        if (!has_next) break;
        item = next;
        g = gn;
        m0 = m0n;
        n0 = n0n;
        A = An;
        B = Bn;
    }
}

// Split-K reduction: C = alpha * sum_s part[s] + bias + beta * C (deterministic order).
__global__ __launch_bounds__(256) void splitk_reduce_k(const float* __restrict__ part, int splits, long MN, int N,
                                                       float* __restrict__ C, long ldc, float alpha, float beta,
                                                       const float* __restrict__ bias) {
    const long stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < MN; i += stride) {
        float s = 0.0f;
        for (int k = 0; k < splits; ++k) s += part[(long)k * MN + i];
        const long r = i / N;
        const int c = (int)(i - r * N);
        float a = alpha * s;
        if (bias) a += bias[c];
        float* cp = C + r * ldc + c;
        if (beta != 0.0f) a += beta * *cp;
        *cp = a;
    }
}

// Column sums, optionally per group of rows: out[g*N + c] (+)= sum over the
// rows of group g of X[r][c] (bias gradients: colsum_raw of
// rust/src/cuda/mod.rs:642-669 and the per-expert db1 of model.rs:432-440).
// Pass 1: a block sums 64 columns over one row slice, its four waves taking
// every fourth row with four independent accumulators; pass 2 sums the slices.
// Every sum has a fixed order, so results are deterministic.
constexpr int CS_SLICE = 128;  // target rows per slice
__global__ __launch_bounds__(256) void colsum_part_k(const float* __restrict__ X, long rows, int N, long ldx,
                                                     const int* __restrict__ goff, float* __restrict__ part,
                                                     int nslices) {
    // grid: (ceil(N / 64), nslices, groups)
    __shared__ float red[4][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + lane;
    const int g = blockIdx.z;
    long lo = 0, hi = rows;
    if (goff) {
        lo = goff[g];
        hi = goff[g + 1];
    }
    const long per = (hi - lo + nslices - 1) / nslices;
    const long a = lo + (long)blockIdx.y * per;
    const long b = min(hi, a + per);
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    if (c < N) {
        long r = a + w;
        for (; r + 12 < b; r += 16) {
            s0 += X[r * ldx + c];
            s1 += X[(r + 4) * ldx + c];
            s2 += X[(r + 8) * ldx + c];
            s3 += X[(r + 12) * ldx + c];
        }
        for (; r < b; r += 4) s0 += X[r * ldx + c];
    }
    red[w][lane] = (s0 + s1) + (s2 + s3);
    __syncthreads();
    if (w == 0 && c < N)
        part[((long)g * nslices + blockIdx.y) * N + c] = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
}

__global__ __launch_bounds__(256) void colsum_fin_k(const float* __restrict__ part, int nslices, int N,
                                                    float* __restrict__ out, int accumulate) {
    // grid: (ceil(N / 64), groups)
    __shared__ float red[4][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + lane;
    const long g = blockIdx.y;
    float s = 0.0f;
    if (c < N)
        for (int k = w; k < nslices; k += 4) s += part[(g * nslices + k) * N + c];
    red[w][lane] = s;
    __syncthreads();
    if (w == 0 && c < N) {
        const float t = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
        const long o = g * N + c;
        out[o] = accumulate ? out[o] + t : t;
    }
}

// ---------------------------------------------------------------- host side

static int ws_check(const Ws& ws, size_t floats, const char* name) {
    if (floats == 0) return ASCA_OK;
    if (!ws.p || ws.floats < floats)
        return fail(ASCA_ERR_INVALID, "%s: workspace of %zu floats, %zu needed", name, ws.floats, floats);
    return ASCA_OK;
}

template <bool TA, bool TB, int EPI, bool VEC, int WM = 2, int WN = 2, int TNW = 4, bool DMA = false>
static int launch_gemm_t(const GemmArgs& a, dim3 grid, hipStream_t st) {
    constexpr size_t lds =
        DMA ? (size_t)DMA_STAGES * dma_stage_bytes<WN>()
            : 2 * (size_t)(tile_floats<!TA, 64 * WM>() + tile_floats<TB, 16 * TNW * WN>()) * sizeof(float);
    if (int arc = allow_lds(reinterpret_cast<const void*>(&gemm_k<TA, TB, EPI, VEC, WM, WN, TNW, DMA>), lds)) return arc;
    hipLaunchKernelGGL((gemm_k<TA, TB, EPI, VEC, WM, WN, TNW, DMA>), grid, dim3(64 * WM * WN), lds, st, a);
    return ASCA_OK;
}

// Fraction of the block slots used over the rounds a launch of `tiles` blocks
// takes, `per_cu` blocks resident per CU.
static double round_fill(long tiles, int per_cu) {
    const long slots = (long)per_cu * (cu_count() > 0 ? cu_count() : 256);
    const long rounds = (tiles + slots - 1) / slots;
    return rounds ? (double)tiles / (double)(rounds * slots) : 1.0;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <bool TA, bool TB, int WM, int WN>
static int launch_batched_t(const GemmArgs& a, long items, hipStream_t st) {
    constexpr size_t lds =
        2 * (size_t)(tile_floats<!TA, 64 * WM>() + tile_floats<TB, 64 * WN>()) * sizeof(float);
    if (int arc = allow_lds(reinterpret_cast<const void*>(&gemm_batched_k<TA, TB, WM, WN>), lds)) return arc;
    // two resident blocks per CU, each walking items with a grid stride
    const long cap = 2L * (cu_count() > 0 ? cu_count() : 256);
    const unsigned grid = (unsigned)(items < cap ? items : cap);
    hipLaunchKernelGGL((gemm_batched_k<TA, TB, WM, WN>), dim3(grid), dim3(64 * WM * WN), lds, st, a);
    return ASCA_OK;
}

// Validates and launches one (possibly grouped) GEMM.  `m_total`: for gmode 1,
// the total rows over all groups (bounds the grid).
int gemm_launch(int ta, int tb, int epi, GemmArgs a, long m_total, hipStream_t st, const char* name) {
    if (a.M < 0 || a.N < 0 || a.K < 0) return fail(ASCA_ERR_INVALID, "%s: negative shape", name);
    if (a.gmode == 1 && ta) return fail(ASCA_ERR_INVALID, "%s: grouped rows need a non-transposed A", name);
    if (a.resid && (epi != EPI_STORE || a.k_per_split > 0))
        return fail(ASCA_ERR_UNSUPPORTED, "%s: residual input needs the plain epilogue without split-K", name);
    if (a.gmode == 2 && (!ta || tb)) return fail(ASCA_ERR_INVALID, "%s: grouped K needs A^T and B", name);
    if (epi == EPI_SILU && (ta || tb)) return fail(ASCA_ERR_UNSUPPORTED, "%s: SiLU epilogue is NN only", name);
    if (epi == EPI_SILU_BWD && (ta || !tb)) return fail(ASCA_ERR_UNSUPPORTED, "%s: SiLU-bwd epilogue is NT only", name);
    if (a.gmode == 3 && (a.a_rows || a.b_rows || a.c_rows || epi != EPI_STORE))
        return fail(ASCA_ERR_UNSUPPORTED, "%s: batched products take no row indirection or fused epilogue", name);
    const bool vec = (a.lda % 4 == 0) && (a.ldb % 4 == 0) && (a.ldc % 4 == 0) && (a.ld_aux % 4 == 0) &&
                     aligned16(a.A) && aligned16(a.B) && aligned16(a.C) && (!a.aux || aligned16(a.aux)) &&
                     (!a.aux_out || aligned16(a.aux_out)) && (a.a_gs % 4 == 0) && (a.b_gs % 4 == 0) &&
                     (a.c_gs % 4 == 0) && (a.c_split_stride % 4 == 0);
    // batched per-chunk products with at most 64 rows use 64 x 128 tiles
    const int wm = (a.gmode == 3 && vec && a.M <= 64) ? 1 : 2;
    const int wn = 2;  // a 64 x 64 tile needs 8 staged float4 per operand per lane and spills
    // block count for a block-tile width bn
    auto count = [&](int bn) -> long {
        const long tn = (a.N + bn - 1) / bn, tm = (a.M + 64 * wm - 1) / (64 * wm);
        const long splits = a.gmode == 0 && a.k_per_split > 0 ? (a.K + a.k_per_split - 1) / a.k_per_split : 1;
        if (a.gmode == 1) return ((m_total + GM_BM - 1) / GM_BM + a.ngroups) * tn;
        if (a.gmode == 2 || a.gmode == 3) return (long)a.ngroups * tm * tn;
        return tm * tn * splits;
    };
    // 128 x 64 tiles when the 128 x 128 grid would leave a mostly idle last
    // round.  Measured per-flop efficiency of the narrow tile against the wide
    // one: ~0.8 with two blocks per CU (NN, NT), ~0.95 with three (A^T)
    const size_t lds64 = 2 * (size_t)(ta ? GM_BK * 128 : 128 * GM_LDK) * sizeof(float) +
                         2 * (size_t)(tb ? 64 * GM_LDK : GM_BK * 64) * sizeof(float);
    // resident narrow blocks per CU: LDS, and registers (the A^T variants fit
    // three waves per SIMD, the others two)
    const int per_cu64 = (int)min((size_t)(ta ? 3 : 2), (size_t)(160 * 1024) / lds64);
    const bool narrow =
        vec && wm == 2 && a.gmode != 3 &&
        round_fill(count(64), per_cu64) * (per_cu64 >= 3 ? 0.95 : 0.8) > round_fill(count(128), 2);
    // Direct-to-LDS 128 x 256 tiles (one 8-wave block per CU) where every
    // operand float4 is whole (k-contiguous operands need K in multiples of 4,
    // mn-contiguous ones M or N) and the grid (tiles x K splits) fills whole
    // rounds of the CUs.  Measured against the 128 x 128 register-staged tile:
    // 5-9% faster on plain products with full rounds (16384 x {1536, 512} x 512
    // NN and NT, 4096^3) and on the grouped-K expert weight gradients, and on
    // the split-K weight gradients (512x1536x16384 TN, ten splits: 272 -> 243
    // us; the configs[3] training step 21.55 -> 20.83 ms); slower with a partly
    // empty last round and on the grouped-row products.
    const bool kc_any = !ta || tb;
    const bool dma_ops = vec && (!kc_any || a.K % 4 == 0) && (!ta || a.M % 4 == 0) && (tb || a.N % 4 == 0) &&
                         a.N >= 4 && (!ta || a.M >= 4);
    const bool dma_ok = dma_ops && (a.gmode == 0 || a.gmode == 2);
    auto count_dma = [&]() -> long {
        const long tn = (a.N + 255) / 256, tm = (a.M + 127) / 128;
        const long sp = a.gmode == 0 && a.k_per_split > 0 ? (a.K + a.k_per_split - 1) / a.k_per_split : 1;
        return a.gmode == 2 ? (long)a.ngroups * tm * tn : tm * tn * sp;
    };
    const bool dma = dma_ok && wm == 2 && round_fill(count_dma(), 1) >= 0.9;
    // otherwise the same loads on a 128 x 128 tile (4 waves, two blocks per CU)
    // for the grouped-row expert products and the other plain products
    // (measured: MoE forward 466 -> 439 us, backward 903 -> 840 us, the
    // 16384x256x512 head 52 -> 48 us, 512x1536x16384 TN split ten ways on
    // this tile 272 -> 258 us)
    const bool dma128 = !dma && dma_ops && wm == 2 && (a.gmode == 1 || a.gmode == 0);
    const int bn = dma ? 256 : dma128 ? 128 : narrow ? 64 : 128;
    a.tiles_n = (a.N + bn - 1) / bn;
    a.tiles_m = (a.M + 64 * wm - 1) / (64 * wm);
    long blocks;
    if (a.gmode == 1)
        blocks = ((m_total + GM_BM - 1) / GM_BM + a.ngroups) * a.tiles_n;
    else if (a.gmode == 2 || a.gmode == 3)
        blocks = (long)a.ngroups * a.tiles_m * a.tiles_n;
    else
        blocks = (long)a.tiles_m * a.tiles_n;
    if (blocks == 0 || a.N == 0) return ASCA_OK;
    if (blocks > 0x7fffffffL) return fail(ASCA_ERR_INVALID, "%s: grid too large", name);
    int rc = pre_launch(name);
    if (rc) return rc;
    const dim3 grid((unsigned)blocks, (unsigned)(a.gmode == 0 && a.k_per_split > 0 ? (a.K + a.k_per_split - 1) / a.k_per_split : 1));
    if (a.gmode != 0 || a.k_per_split <= 0) a.k_per_split = a.K;
#define ASCA_GEMM_CASE(TA_, TB_, EPI_)                                                                  \
    if (ta == TA_ && tb == TB_ && epi == EPI_)                                                          \
        rc = !vec ? launch_gemm_t<TA_, TB_, EPI_, false>(a, grid, st)                                   \
             : dma    ? launch_gemm_t<TA_, TB_, EPI_, true, 2, 4, 4, true>(a, grid, st)                 \
             : dma128 ? launch_gemm_t<TA_, TB_, EPI_, true, 2, 2, 4, true>(a, grid, st)                 \
             : narrow ? launch_gemm_t<TA_, TB_, EPI_, true, 2, 2, 2>(a, grid, st)                       \
                      : launch_gemm_t<TA_, TB_, EPI_, true>(a, grid, st);                                \
    else
#define ASCA_GEMM_SMALL(TA_, TB_)                                                                       \
    if (ta == TA_ && tb == TB_)                                                                         \
        rc = launch_gemm_t<TA_, TB_, EPI_STORE, true, 1, 2>(a, grid, st);                               \
    else
#define ASCA_GEMM_BATCHED(TA_, TB_)                                                                     \
    if (ta == TA_ && tb == TB_)                                                                         \
        rc = wm == 1 ? launch_batched_t<TA_, TB_, 1, 2>(a, blocks, st)                                  \
                     : launch_batched_t<TA_, TB_, 2, 2>(a, blocks, st);                                 \
    else
    if (a.gmode == 3 && vec && a.K > 0) {
        ASCA_GEMM_BATCHED(0, 0)
        ASCA_GEMM_BATCHED(1, 0)
        ASCA_GEMM_BATCHED(0, 1)
        ASCA_GEMM_BATCHED(1, 1)
        rc = fail(ASCA_ERR_UNSUPPORTED, "%s: no kernel for this variant", name);
        if (rc) return rc;
        return post_launch(name);
    }
#undef ASCA_GEMM_BATCHED
    if (wm == 1) {
        ASCA_GEMM_SMALL(0, 0)
        ASCA_GEMM_SMALL(1, 0)
        ASCA_GEMM_SMALL(0, 1)
        ASCA_GEMM_SMALL(1, 1)
        rc = fail(ASCA_ERR_UNSUPPORTED, "%s: no kernel for this variant", name);
        if (rc) return rc;
        return post_launch(name);
    }
#undef ASCA_GEMM_SMALL
    ASCA_GEMM_CASE(0, 0, EPI_STORE)
    ASCA_GEMM_CASE(1, 0, EPI_STORE)
    ASCA_GEMM_CASE(0, 1, EPI_STORE)
    ASCA_GEMM_CASE(1, 1, EPI_STORE)
    ASCA_GEMM_CASE(0, 0, EPI_SILU)
    ASCA_GEMM_CASE(0, 1, EPI_SILU_BWD)
    rc = fail(ASCA_ERR_UNSUPPORTED, "%s: no kernel for this variant", name);
#undef ASCA_GEMM_CASE
    if (rc) return rc;
    return post_launch(name);
}

GemmArgs gemm_args() {
    GemmArgs a{};
    a.alpha = 1.0f;
    a.beta = 0.0f;
    return a;
}

// Slices of a column sum: about CS_SLICE rows each (twice as many per group:
// group sizes vary).
static int colsum_slices(long rows, int G, bool grouped) {
    const long avg = grouped ? (2 * rows) / G + 1 : rows;
    const int ns = (int)min((avg + CS_SLICE - 1) / CS_SLICE, 1024L);
    return ns < 1 ? 1 : ns;
}

size_t colsum_ws_floats(long rows, int N, bool grouped, int ngroups) {
    const int G = grouped ? ngroups : 1;
    if (N <= 0 || G <= 0) return 0;
    return (size_t)G * colsum_slices(rows, G, grouped) * N;
}

// Column sums of X (rows x N, ld ldx), per group when goff is given.
int colsum_launch(const float* X, long rows, int N, long ldx, const int* goff, int ngroups, float* out,
                  int accumulate, Ws ws, hipStream_t st) {
    if (N == 0) return ASCA_OK;
    const int G = goff ? ngroups : 1;
    if (G == 0) return ASCA_OK;
    const int cb = (N + 63) / 64;
    const int ns = colsum_slices(rows, G, goff != nullptr);
    int rc = ws_check(ws, (size_t)G * ns * N, "colsum");
    if (rc) return rc;
    float* const part = ws.p;
    rc = pre_launch("colsum");
    if (rc) return rc;
    hipLaunchKernelGGL(colsum_part_k, dim3(cb, ns, G), dim3(256), 0, st, X, rows, N, ldx, goff, part, ns);
    rc = post_launch("colsum");
    if (rc) return rc;
    rc = pre_launch("colsum_fin");
    if (rc) return rc;
    hipLaunchKernelGGL(colsum_fin_k, dim3(cb, G), dim3(256), 0, st, part, ns, N, out, accumulate);
    return post_launch("colsum_fin");
}

// ---------------------------------------------------------------------------
// Skinny products with n <= 16 output columns (the gate projection, n = 2H):
// the 16-wide MFMA output tile matches them, where a 128-wide block tile of
// the general kernel would multiply mostly padding.
//
// Forward Y (T x n) = X (T x K) W (K x n) + b: one wave per 16 rows.  Lane
// (i = l % 16, q = l / 16) supplies A = X[row i][16 j + 4 q + e] from one
// 16-byte load per 16-k group j (e = 0..3 are four MFMA k-steps: the k index
// is permuted inside each group of 16, which the sum does not see) and keeps
// the matching B = W[16 j + 4 q + e][i] for the whole K in registers.
template <int KT>  // K = 16 KT
__global__ __launch_bounds__(256) void skinny_fwd_k(const float* __restrict__ X, long ldx, const float* __restrict__ W,
                                                    const float* __restrict__ b, float* __restrict__ Y, long T, int n) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const long r0 = ((long)blockIdx.x * 4 + w) * 16;
    if (r0 >= T) return;  // whole wave
    const int i = lane & 15, q = lane >> 4;
    const int ic = min(i, n - 1);
    float wb[4 * KT];
#pragma unroll
    for (int j = 0; j < KT; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float v = W[(long)(16 * j + 4 * q + e) * n + ic];
            wb[4 * j + e] = i < n ? v : 0.0f;
        }
    const float* xr = X + min(r0 + i, T - 1) * ldx + 4 * q;
    float4 xv[KT];
#pragma unroll
    for (int j = 0; j < KT; ++j) xv[j] = *reinterpret_cast<const float4*>(xr + 16 * j);
    // every load above is in flight before the first product (the scheduler
    // would otherwise interleave them with the products, one wait each)
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KT; ++j) {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[j].x, wb[4 * j + 0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[j].y, wb[4 * j + 1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[j].z, wb[4 * j + 2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[j].w, wb[4 * j + 3], acc, 0, 0, 0);
    }
    const float bi = b ? b[ic] : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const long row = r0 + 4 * q + r;
        if (i < n && row < T) Y[row * n + i] = acc[r] + bi;
    }
}

// Weight gradient G (K x n) = X^T D and bias gradient db = column sums of D,
// over T rows.  Wave (tile it, chunk s) reduces rows s*SK_T .. +SK_T into a
// 16 x 16 partial of G (i = 16 it + lane % 16): per MFMA k-step the four lane
// groups q take rows t = 4 m + q, lane (i, q) supplies X[t][16 it + i] and
// D[t][i].  Waves of tile 0 also sum their D values for db.  Partials go to
// part[s][K + 1][16] (row K: db) and skinny_reduce_k adds them in a fixed order.
constexpr int SK_T = 256;  // rows per wave
__global__ __launch_bounds__(256) void skinny_wgrad_k(const float* __restrict__ X, long ldx,
                                                      const float* __restrict__ D, long T, int K, int n,
                                                      float* __restrict__ part) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int it = blockIdx.x;
    const long s = (long)blockIdx.y * 4 + w;
    const long nch = (T + SK_T - 1) / SK_T;
    if (s >= nch) return;  // whole wave
    const int i = lane & 15, q = lane >> 4;
    const int ic = min(i, n - 1);
    const long t0 = s * SK_T;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float dsum = 0.0f;
    constexpr int NM = SK_T / 4;
    constexpr int G = 16;  // k-steps whose loads are issued together
#pragma unroll 1
    for (int m0 = 0; m0 < NM; m0 += G) {
        float av[G], bv[G];
#pragma unroll
        for (int u = 0; u < G; ++u) {
            const long t = t0 + 4 * (m0 + u) + q;
            const long tc = min(t, T - 1);
            const float xa = X[tc * ldx + 16 * it + i];
            const float db = D[tc * n + ic];
            av[u] = t < T ? xa : 0.0f;
            bv[u] = (t < T && i < n) ? db : 0.0f;
        }
        __builtin_amdgcn_sched_barrier(0);  // the group's loads go out together
#pragma unroll
        for (int u = 0; u < G; ++u) {
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], bv[u], acc, 0, 0, 0);
            dsum += bv[u];
        }
    }
    float* ps = part + s * (long)(K + 1) * 16;
#pragma unroll
    for (int r = 0; r < 4; ++r) ps[(16 * it + 4 * q + r) * 16 + i] = acc[r];
    if (it == 0) {
        dsum += __shfl_xor(dsum, 16);
        dsum += __shfl_xor(dsum, 32);
        if (q == 0) ps[K * 16 + i] = dsum;
    }
}

// One wave per output row of the (K + 1) x n result: lane (c = l % 16,
// g = l / 16) adds chunks g, g + 4, ... (independent loads, all in flight),
// then the four lane groups are added (a fixed order).
__global__ __launch_bounds__(256) void skinny_reduce_k(const float* __restrict__ part, long nch, int K, int n,
                                                       float* __restrict__ G, float* __restrict__ db) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row > K) return;  // whole wave
    const int c = lane & 15, g = lane >> 4;
    float acc = 0.0f;
    for (long s = g; s < nch; s += 4) acc += part[(s * (K + 1) + row) * 16 + c];
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    if (g == 0 && c < n) {
        if (row < K)
            G[row * n + c] = acc;
        else if (db)
            db[c] = acc;
    }
}

static bool skinny_ok(const float* X, long ldx, int K, int n) {
    return n >= 1 && n <= 16 && (K == 128 || K == 256 || K == 512) && ldx % 4 == 0 &&
           (reinterpret_cast<uintptr_t>(X) & 15) == 0;
}

int skinny_fwd_launch(const float* X, long ldx, const float* W, const float* b, float* Y, long T, int K, int n,
                      hipStream_t st) {
    if (T <= 0 || n <= 0) return ASCA_OK;
    if (!skinny_ok(X, ldx, K, n)) {
        GemmArgs a = gemm_args();
        a.A = X;
        a.lda = ldx;
        a.B = W;
        a.ldb = n;
        a.C = Y;
        a.ldc = n;
        a.M = (int)T;
        a.N = n;
        a.K = K;
        a.bias = b;
        return gemm_launch(0, 0, EPI_STORE, a, T, st, "skinny_fwd");
    }
    int rc = pre_launch("skinny_fwd");
    if (rc) return rc;
    const dim3 grid((unsigned)((T + 63) / 64));
    if (K == 512)
        hipLaunchKernelGGL(skinny_fwd_k<32>, grid, dim3(256), 0, st, X, ldx, W, b, Y, T, n);
    else if (K == 256)
        hipLaunchKernelGGL(skinny_fwd_k<16>, grid, dim3(256), 0, st, X, ldx, W, b, Y, T, n);
    else
        hipLaunchKernelGGL(skinny_fwd_k<8>, grid, dim3(256), 0, st, X, ldx, W, b, Y, T, n);
    return post_launch("skinny_fwd");
}

size_t skinny_wgrad_ws_floats(long T, int K, int n) {
    if (n <= 0 || K <= 0) return 0;
    const size_t fallback = max(gemm_ws_floats(K, n, (int)min(T, 0x7fffffffL)), colsum_ws_floats(T, n, false, 0));
    const long nch = (max(T, 0L) + SK_T - 1) / SK_T;
    return max(fallback, (size_t)nch * (K + 1) * 16);
}

int skinny_wgrad_launch(const float* X, long ldx, const float* D, float* G, float* db, long T, int K, int n,
                        Ws ws, hipStream_t st) {
    if (n <= 0 || K <= 0) return ASCA_OK;
    if (T <= 0 || !skinny_ok(X, ldx, K, n) || K % 16) {
        int rc = gemm_run(1, 0, K, n, (int)T, 1.0f, X, ldx, D, n, 0.0f, G, n, nullptr, ws, st);
        if (rc || !db) return rc;
        return colsum_launch(D, T, n, n, nullptr, 0, db, 0, ws, st);
    }
    const long nch = (T + SK_T - 1) / SK_T;
    int rc = ws_check(ws, (size_t)nch * (K + 1) * 16, "skinny_wgrad");
    if (rc) return rc;
    float* const part = ws.p;
    if ((rc = pre_launch("skinny_wgrad"))) return rc;
    hipLaunchKernelGGL(skinny_wgrad_k, dim3((unsigned)(K / 16), (unsigned)((nch + 3) / 4)), dim3(256), 0, st, X, ldx,
                       D, T, K, n, part);
    if ((rc = post_launch("skinny_wgrad"))) return rc;
    if ((rc = pre_launch("skinny_reduce"))) return rc;
    hipLaunchKernelGGL(skinny_reduce_k, dim3((unsigned)((K + 1 + 3) / 4)), dim3(256), 0, st, part, nch, K, n, G, db);
    return post_launch("skinny_reduce");
}

// Split-K decision of a plain product: split K when the output has too few
// tiles to fill the chip, into as many K ranges as keep the grid within one
// round of two blocks per CU (rounding up gave 512x1536x16384 eleven splits,
// 528 blocks: a second round of 16; ten splits take it 315 -> 277 us).
// Returns the split count and the K range per split.
static int gemm_splits(int M, int N, int K, long* kps_out) {
    const long tiles = (long)((M + GM_BM - 1) / GM_BM) * ((N + GM_BN - 1) / GM_BN);
    const int cus = cu_count() > 0 ? cu_count() : 256;
    int splits = 1;
    if (tiles < cus && K >= 1024) {
        splits = (int)min((long)K / 512, (2L * cus) / tiles);
        if (splits < 1) splits = 1;
    }
    long kps = K;
    if (splits > 1) {
        kps = ((K + splits - 1) / splits + GM_BK - 1) / GM_BK * GM_BK;
        splits = (int)((K + kps - 1) / kps);
    }
    *kps_out = kps;
    return splits;
}

size_t gemm_ws_floats(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    long kps = 0;
    const int splits = gemm_splits(M, N, K, &kps);
    return splits > 1 ? (size_t)splits * M * N : 0;
}

int gemm_check(int trans_a, int trans_b, int M, int N, int K, const float* A, long lda, const float* B, long ldb,
               const float* C, long ldc) {
    if (M < 0 || N < 0 || K < 0) return fail(ASCA_ERR_INVALID, "asca_gemm: negative shape");
    if (M == 0 || N == 0) return ASCA_OK;
    if (!C || (K > 0 && (!A || !B))) return fail(ASCA_ERR_INVALID, "asca_gemm: null pointer");
    const long a_cols = trans_a ? M : K, b_cols = trans_b ? K : N;
    if (lda < a_cols || ldb < b_cols || ldc < N) return fail(ASCA_ERR_INVALID, "asca_gemm: leading dimension too small");
    return ASCA_OK;
}

// C = alpha op(A) op(B) + beta C (+ bias), split-K partials in ws.
int gemm_run(int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A, long lda, const float* B,
             long ldb, float beta, float* C, long ldc, const float* bias, Ws ws, hipStream_t st) {
    if (M == 0 || N == 0) return ASCA_OK;
    GemmArgs a = gemm_args();
    a.A = A;
    a.B = B;
    a.C = C;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.M = M;
    a.N = N;
    a.K = K;
    a.alpha = alpha;
    a.beta = beta;
    a.bias = bias;
    long kps = 0;
    const int splits = K > 0 ? gemm_splits(M, N, K, &kps) : 1;
    if (splits == 1) return gemm_launch(trans_a, trans_b, EPI_STORE, a, M, st, "gemm");
    const long MN = (long)M * N;
    int rc = ws_check(ws, (size_t)splits * MN, "gemm split-K");
    if (rc) return rc;
    float* const part = ws.p;
    GemmArgs s = a;
    s.C = part;
    s.ldc = N;
    s.alpha = 1.0f;
    s.beta = 0.0f;
    s.bias = nullptr;
    s.k_per_split = kps;
    s.c_split_stride = MN;
    rc = gemm_launch(trans_a, trans_b, EPI_STORE, s, M, st, "gemm_splitk");
    if (rc) return rc;
    rc = pre_launch("splitk_reduce");
    if (rc) return rc;
    const int cus = cu_count() > 0 ? cu_count() : 256;
    long blocks = (MN + 255) / 256;
    if (blocks > 4L * cus * 8) blocks = 4L * cus * 8;
    hipLaunchKernelGGL(splitk_reduce_k, dim3((unsigned)blocks), dim3(256), 0, st, part, splits, MN, N, C, ldc, alpha,
                       beta, bias);
    return post_launch("splitk_reduce");
}

// Scratch of asca_gemm_noalloc, the entry point for callers that cannot
// allocate: a static device array of SCRATCH_FLOATS floats (32 MiB), which
// every device the library runs on holds until the process ends.  Its size is
// the most split-K partials can take on gfx950 (256 CUs): gemm_splits keeps
// splits * tiles <= 2 * CUs and a tile covers at most GM_BM x GM_BN outputs,
// so splits * M * N <= 2 * 256 * GM_BM * GM_BN floats; the size check in
// asca_gemm_noalloc stays as a guard.  In host code `scratch` names a
// host-side stand-in, never the device memory: its device address comes from
// hipGetSymbolAddress, once per device at asca_init (with that device
// current), and only that address is used.
constexpr size_t SCRATCH_FLOATS = (size_t)2 * 256 * GM_BM * GM_BN;
static __device__ __align__(256) float scratch[SCRATCH_FLOATS];
static float* g_scratch_dev[64] = {};

int noalloc_scratch_init(int device) {
    if (device < 0 || device >= 64) return fail(ASCA_ERR_INVALID, "device %d out of range", device);
    if (g_scratch_dev[device]) return ASCA_OK;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return fail(ASCA_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    g_scratch_dev[device] = reinterpret_cast<float*>(p);
    return ASCA_OK;
}

}  // namespace asca

using namespace asca;

extern "C" {

int asca_gemm_ws_bytes(int trans_a, int trans_b, int M, int N, int K, size_t* bytes) {
    (void)trans_a;
    (void)trans_b;
    if (!bytes) return fail(ASCA_ERR_INVALID, "null output pointer");
    if (M < 0 || N < 0 || K < 0) return fail(ASCA_ERR_INVALID, "asca_gemm_ws_bytes: negative shape");
    *bytes = gemm_ws_floats(M, N, K) * sizeof(float);
    return ASCA_OK;
}

int asca_gemm_ws(int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A, long lda, const float* B,
                 long ldb, float beta, float* C, long ldc, const float* bias, void* ws, size_t ws_bytes,
                 void* stream) {
    int rc = gemm_check(trans_a, trans_b, M, N, K, A, lda, B, ldb, C, ldc);
    if (rc || M == 0 || N == 0) return rc;
    return gemm_run(trans_a, trans_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias,
                    Ws{reinterpret_cast<float*>(ws), ws_bytes / sizeof(float)}, as_stream(stream));
}

// The reference's matmul takes no workspace: split-K partials come from the
// stream-ordered allocator on the call's stream and go back to it behind the
// reduction, so calls on different streams never share them.
int asca_gemm(int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A, long lda, const float* B,
              long ldb, float beta, float* C, long ldc, const float* bias, void* stream) {
    int rc = gemm_check(trans_a, trans_b, M, N, K, A, lda, B, ldb, C, ldc);
    if (rc || M == 0 || N == 0) return rc;
    const hipStream_t st = as_stream(stream);
    const size_t need = gemm_ws_floats(M, N, K);
    StreamScratch sc;
    if ((rc = sc.get(need, st))) return rc;
    rc = gemm_run(trans_a, trans_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias, sc.ws, st);
    const int rf = sc.release(st);
    return rc ? rc : rf;
}

// asca_gemm whose split-K partials live in the static scratch: allocates
// nothing.  Calls that overlap on one device share that scratch and race.
int asca_gemm_noalloc(int trans_a, int trans_b, int M, int N, int K, float alpha, const float* A, long lda,
                      const float* B, long ldb, float beta, float* C, long ldc, const float* bias, void* stream) {
    int rc = gemm_check(trans_a, trans_b, M, N, K, A, lda, B, ldb, C, ldc);
    if (rc || M == 0 || N == 0) return rc;
    if ((rc = ensure_device())) return rc;
    const size_t need = gemm_ws_floats(M, N, K);
    if (need > SCRATCH_FLOATS)
        return fail(ASCA_ERR_INVALID,
                    "asca_gemm_noalloc: the split-K partials of %dx%dx%d need %zu bytes, the static scratch holds "
                    "%zu (use asca_gemm_ws)",
                    M, N, K, need * sizeof(float), SCRATCH_FLOATS * sizeof(float));
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || !g_scratch_dev[dev])
        return fail(ASCA_ERR_NOT_INIT, "asca_gemm_noalloc: no static scratch address for device %d", dev);
    return gemm_run(trans_a, trans_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, bias,
                    Ws{g_scratch_dev[dev], SCRATCH_FLOATS}, as_stream(stream));
}

int asca_colsum_ws_bytes(long rows, int cols, size_t* bytes) {
    if (!bytes) return fail(ASCA_ERR_INVALID, "null output pointer");
    if (rows < 0 || cols < 0) return fail(ASCA_ERR_INVALID, "asca_colsum_ws_bytes: negative shape");
    *bytes = colsum_ws_floats(rows, cols, false, 0) * sizeof(float);
    return ASCA_OK;
}

int asca_colsum_ws(const float* X, long rows, int cols, float* out, int accumulate, void* ws, size_t ws_bytes,
                   void* stream) {
    if (rows < 0 || cols < 0) return fail(ASCA_ERR_INVALID, "asca_colsum: negative shape");
    if (cols == 0) return ASCA_OK;
    if (!out || (rows > 0 && !X)) return fail(ASCA_ERR_INVALID, "asca_colsum: null pointer");
    return colsum_launch(X, rows, cols, cols, nullptr, 0, out, accumulate,
                         Ws{reinterpret_cast<float*>(ws), ws_bytes / sizeof(float)}, as_stream(stream));
}

int asca_colsum(const float* X, long rows, int cols, float* out, int accumulate, void* stream) {
    if (rows < 0 || cols < 0) return fail(ASCA_ERR_INVALID, "asca_colsum: negative shape");
    if (cols == 0) return ASCA_OK;
    if (!out || (rows > 0 && !X)) return fail(ASCA_ERR_INVALID, "asca_colsum: null pointer");
    const hipStream_t st = as_stream(stream);
    StreamScratch sc;
    int rc = sc.get(colsum_ws_floats(rows, cols, false, 0), st);
    if (rc) return rc;
    rc = colsum_launch(X, rows, cols, cols, nullptr, 0, out, accumulate, sc.ws, st);
    const int rf = sc.release(st);
    return rc ? rc : rf;
}

}  // extern "C"
