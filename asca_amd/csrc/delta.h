// Internals shared by the delta-rule translation units (delta.hip: the
// recurrent kernels for every dh other than 64, on eight-lane column groups, and
// the entry points; delta_ut64.hip: dh = 64 in the blocked form).
#pragma once
#include "common.h"

namespace asca {

// Workspace of one forward / backward pair (asca_delta_ws_bytes):
//  * sk: the recurrent kernels' per-step S_{t-1}^T k_t vectors (the blocked
//    form's u rows), layout of v;
//  * ckpt: per unit (h*B + b), nslots = ceil(T/ck) + 1 states of dh^2 floats
//    (the recurrent kernels store S^T, element (a, i) at i*dh + a; the blocked
//    form its own tile order): slot j is the state before step j*ck for
//    j < ceil(T/ck), the last slot the state after step T-1;
//  * rec: the blocked form's per-block records.
// The forward writes it; the backward only reads it (a column-split backward
// keeps its partial sums in scratch of its own), so several backwards may read
// one forward's workspace at once.
struct DeltaWs {
    float* sk;
    float* ckpt;
    float* rec;     // dh = 64 blocked form: per unit and 16-step block, K K^T, Q K^T, T, M, Gamma, gate vectors
    int ck;
    int nslots;
    int cs;
    size_t bytes;
};

// Sum of the 2*CK per-step partials (dalpha of step j, dbeta of step j) over
// all 64 lanes, given y[j] = their first transposed level (tsum32: lanes < 32
// hold the dalpha pair sum of step j, lanes >= 32 the dbeta one); two more
// swap/DPP levels on halving value sets, then a butterfly over the lanes left;
// the totals go to red_ab[(j*W + w)*2 + {0: dalpha, 1: dbeta}].
template <int CK, int W>
ASCA_DEV void cross_step_sum(const float (&y)[CK], float* __restrict__ red_ab, int w, int lane) {
    constexpr int K = 2 * CK;
    // lane holds y[i] = total over lane bit 5 of x[i + (bit5 ? K/2 : 0)]
    if constexpr (K / 2 >= 2) {
        float z[K / 4];
#pragma unroll
        for (int i = 0; i < K / 4; ++i) z[i] = tsum16(y[i], y[i + K / 4]);
        if constexpr (K / 4 >= 2) {
            const bool b3 = (lane & 8) != 0;
            float u[K / 8];
#pragma unroll
            for (int i = 0; i < K / 8; ++i) {
                const float keep = b3 ? z[i + K / 8] : z[i];
                const float send = b3 ? z[i] : z[i + K / 8];
                u[i] = keep + dpp<DPP_ROW_ROR8>(send);
            }
#pragma unroll
            for (int i = 0; i < K / 8; ++i) {
                const float tot = group_sum<8>(u[i]);
                const int idx = i + (b3 ? K / 8 : 0) + ((lane & 16) ? K / 4 : 0) + ((lane & 32) ? K / 2 : 0);
                if ((lane & 7) == 0) red_ab[((idx % CK) * W + w) * 2 + idx / CK] = tot;
            }
        } else {
            const float tot = group_sum<16>(z[0]);
            const int idx = ((lane & 16) ? K / 4 : 0) + ((lane & 32) ? K / 2 : 0);
            if ((lane & 15) == 0) red_ab[((idx % CK) * W + w) * 2 + idx / CK] = tot;
        }
    } else {
        const float tot = add_xor16(group_sum<16>(y[0]));
        const int idx = (lane & 32) ? K / 2 : 0;
        if ((lane & 31) == 0) red_ab[((idx % CK) * W + w) * 2 + idx / CK] = tot;
    }
}

// dh = 64: the blocked (UT) form on the matrix cores (delta_ut64.hip), used for
// every dh = 64 shape with one block per unit (ws.cs == 1).  Its workspace: the
// u rows in `sk` (per unit and D64_BLK-step block, as the forward's wave tiles,
// T rounded up to whole blocks), the state before every other block (every
// D64_CK steps) and the final state in `ckpt`, per block a record of D64_REC
// floats in `rec`, all written by the forward and read by the backward.  Any
// pointer alignment.
constexpr int D64_BLK = 16;
constexpr int D64_CK = 2 * D64_BLK;
constexpr int D64_REC = 1344;
int launch_ut_fwd64(const float* q, const float* k, const float* v, const float* alpha, const float* beta, float* o,
                    const DeltaWs& ws, int B, int T, int H, hipStream_t st);
int launch_ut_bwd64(bool fused, const float* q, const float* k, const float* v, const float* alpha,
                    const float* beta, const float* d_o, const DeltaWs& ws, const float* qn, const float* kn,
                    float* gq, float* gk, float* gv, long ldx, float* ga, float* gb, long ldg, int B, int T, int H,
                    hipStream_t st);

}  // namespace asca
