"""The entry point that allocates nothing (asca_gemm_noalloc: split-K
partials in the library's static device scratch) against asca_gemm, through
the C ABI: two calls in a row, the second on a smaller product, each
bit-identical to asca_gemm and within the forward bar of a float64 product."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FWD_TOL = 2e-5


def test_gemm_noalloc_matches_gemm_on_two_calls(orc, g):
    from asca_amd import _lib
    from asca_amd.gpu import DevBuf, _vp

    rng = np.random.default_rng(77)
    # both split K (too few output tiles for the chip), the second is smaller
    for (M, N, K) in ((512, 1536, 16384), (256, 512, 8192)):
        wsb = C.c_size_t()
        _lib.call("asca_gemm_ws_bytes", 1, 0, M, N, K, C.byref(wsb))
        print(f"[noalloc] TN {M}x{N}x{K}: split-K partials {wsb.value} B", flush=True)
        assert 0 < wsb.value <= 64 << 20
        x = rng.standard_normal((K, M)).astype(np.float32)
        d = rng.standard_normal((K, N)).astype(np.float32)
        bias = rng.standard_normal(N).astype(np.float32)
        bx, bd, bb = DevBuf.from_host(x), DevBuf.from_host(d), DevBuf.from_host(bias)
        c1, c2 = DevBuf(M * N * 4), DevBuf(M * N * 4)
        _lib.call("asca_gemm", 1, 0, M, N, K, 0.5, _vp(bx), M, _vp(bd), N, 0.0, _vp(c1), N, _vp(bb), None)
        _lib.call("asca_gemm_noalloc", 1, 0, M, N, K, 0.5, _vp(bx), M, _vp(bd), N, 0.0, _vp(c2), N, _vp(bb), None)
        _lib.call("asca_sync")
        want, got = c1.to_host((M, N)), c2.to_host((M, N))
        np.testing.assert_array_equal(got, want)
        ref = 0.5 * (x.astype(np.float64).T @ d.astype(np.float64)) + bias
        assert orc.rel_err(got, ref) <= FWD_TOL
        for b in (bx, bd, bb, c1, c2):
            b.free()
