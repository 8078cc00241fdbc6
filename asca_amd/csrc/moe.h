// Internal interface of the MoE backward halves (moe.hip) for the training
// step (model.hip).  Not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

#include "runtime.h"

namespace asca {

// dpre (T x d_ff, expert-sorted rows) and dxn (T x d, token rows) from dout.
int moe_bwd_data(const float* w1, const float* w2, const float* pre, const int32_t* perm, const int32_t* offsets,
                 const float* dout, int T, int d, int d_ff, int E, float* dxn, float* dpre_ws, hipStream_t st);
// dW1, db1, dW2, db2 from dout and dpre (written by moe_bwd_data); ws holds
// the column-sum partials (moe_bwd_weights_ws_floats).
int moe_bwd_weights(const float* xn, const float* hidden, const int32_t* perm, const int32_t* offsets,
                    const float* dout, const float* dpre_ws, int T, int d, int d_ff, int E, float* dw1, float* db1,
                    float* dw2, float* db2, int accumulate, Ws ws, hipStream_t st);
size_t moe_bwd_weights_ws_floats(int T, int d, int d_ff, int E);

}  // namespace asca
