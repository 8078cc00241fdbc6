// Gated delta rule at dh = 64, f32: the backward variants off the hot path
// (the raw gradients, and the fused ones on rows not aligned to 16 bytes), in a
// translation unit of their own so that they keep the default instruction
// scheduler (the hot path's setting does not compile them).
#include "ut64_kernels.h"

namespace asca {

int launch_ut_bwd64_other(const ut64::BArgs& a, int units, bool fused, bool al, hipStream_t st) {
    if (fused) return launch_ut_bwd64_t<true, false>(a, units, st);
    return al ? launch_ut_bwd64_t<false, true>(a, units, st) : launch_ut_bwd64_t<false, false>(a, units, st);
}

}  // namespace asca
