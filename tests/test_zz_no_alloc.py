"""The entry point that allocates nothing (asca_gemm_noalloc: split-K
partials in the library's static device scratch) against asca_gemm, through
the C ABI: two calls in a row, the second on a smaller product, each
bit-identical to asca_gemm and within the forward bar of a float64 product;
the device's free memory unchanged across such calls (and, as a control, an
asca_gemm on a new stream visibly allocating); the scratch's size bounding the
partials of every product."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FWD_TOL = 2e-5
SCRATCH_BYTES = 2 * 256 * 128 * 128 * 4   # the static scratch: the split-K bound on gfx950


def _hip_free_bytes():
    """hipMemGetInfo's free bytes from the HIP runtime the library uses."""
    hip = C.CDLL("libamdhip64.so.7")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def test_gemm_noalloc_matches_gemm_on_two_calls(orc, g):
    from asca_amd import _lib
    from asca_amd.gpu import DevBuf, _vp

    rng = np.random.default_rng(77)
    # both split K (too few output tiles for the chip), the second is smaller
    for (M, N, K) in ((512, 1536, 16384), (256, 512, 8192)):
        wsb = C.c_size_t()
        _lib.call("asca_gemm_ws_bytes", 1, 0, M, N, K, C.byref(wsb))
        print(f"[noalloc] TN {M}x{N}x{K}: split-K partials {wsb.value} B", flush=True)
        assert 0 < wsb.value <= SCRATCH_BYTES
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


def test_gemm_noalloc_allocates_nothing(g):
    from asca_amd import _lib
    from asca_amd.gpu import DevBuf, _vp

    M, N, K = 512, 1536, 16384     # split K: 30 MiB of partials
    bx, bd, c = DevBuf(K * M * 4), DevBuf(K * N * 4), DevBuf(M * N * 4)
    args = (1, 0, M, N, K, 1.0, _vp(bx), M, _vp(bd), N, 0.0, _vp(c), N, None, None)
    _lib.call("asca_gemm_noalloc", *args)   # code objects loaded, nothing pending
    _lib.call("asca_sync")
    before = _hip_free_bytes()
    for _ in range(3):
        _lib.call("asca_gemm_noalloc", *args)
    _lib.call("asca_sync")
    after = _hip_free_bytes()
    print(f"[noalloc] device free bytes {before} -> {after}", flush=True)
    assert after == before
    # control: asca_gemm on a stream of its own takes that stream's scratch (the
    # library's pools released first, so the allocation cannot reuse memory they keep)
    _lib.call("asca_pool_release")
    base = _hip_free_bytes()
    sp = C.c_void_p()
    _lib.call("asca_stream_create", C.byref(sp))
    _lib.call("asca_gemm", *args[:-1], sp)
    _lib.call("asca_stream_sync", sp)
    ctrl = _hip_free_bytes()
    print(f"[noalloc] asca_gemm on a new stream: free bytes {base} -> {ctrl}", flush=True)
    assert ctrl < base
    _lib.call("asca_stream_destroy", sp)
    for b in (bx, bd, c):
        b.free()


def test_split_k_partials_never_exceed_the_static_scratch():
    # CPU-side sizing (asca_gemm_ws_bytes needs no device): the shapes that split
    # most, in every transpose case, stay within the static scratch
    from asca_amd import _lib

    worst = 0
    for ta in (0, 1):
        for tb in (0, 1):
            for M in (128, 256, 512, 1000, 1024, 2048):
                for N in (128, 384, 1536, 2048, 4096):
                    for K in (1024, 16384, 1 << 20):
                        wsb = C.c_size_t()
                        _lib.call("asca_gemm_ws_bytes", ta, tb, M, N, K, C.byref(wsb))
                        worst = max(worst, wsb.value)
    print(f"[noalloc] largest split-K partials {worst} B of {SCRATCH_BYTES}", flush=True)
    assert 0 < worst <= SCRATCH_BYTES
