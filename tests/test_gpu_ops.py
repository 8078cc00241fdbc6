"""GPU parity of the rows around the delta block: MFMA GEMM, RMSNorm fwd/bwd,
hash routing + bucketing, row gather/scatter, cross-entropy, AdamW and the
hash-MoE forward/backward, all through the C ABI (asca_amd.gpu ->
libasca_hip.so) against the CPU oracle on the same seeded inputs.

Bars: forward outputs <= 2e-5 and gradients <= 1e-4 as max|gpu-cpu|/max|cpu|
(rust/src/main.rs:1021-1029); routing, bucketing and gather/scatter bit-exact;
AdamW bit-exact (the element update is the CPU's operation sequence).
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FWD_TOL = 2e-5
GRAD_TOL = 1e-4


def test_mfma_16x16x4_lane_layout(g):
    from asca_amd import _lib

    out = np.zeros((16, 64), dtype=np.float32)
    _lib.call("asca_selftest_wave", out.ctypes.data_as(C.c_void_p))
    lane = np.arange(64)
    a = ((lane * 7) % 13 - 6).astype(np.float64)
    b = ((lane * 5) % 11 - 5).astype(np.float64)
    # operand layout: lane l holds A[l % 16][l // 16] and B[l // 16][l % 16]
    A = np.zeros((16, 4))
    Bm = np.zeros((4, 16))
    A[lane % 16, lane // 16] = a
    Bm[lane // 16, lane % 16] = b
    D = A @ Bm
    # result layout: register r of lane l holds D[4 (l // 16) + r][l % 16]
    for r in range(4):
        np.testing.assert_array_equal(out[10 + r], D[4 * (lane // 16) + r, lane % 16])


def _ref_gemm(a, b, ta, tb, alpha, beta, c, bias):
    A = a.astype(np.float64).T if ta else a.astype(np.float64)
    Bm = b.astype(np.float64).T if tb else b.astype(np.float64)
    r = alpha * (A @ Bm)
    if bias is not None:
        r = r + bias.astype(np.float64)
    if beta != 0.0:
        r = r + beta * c.astype(np.float64)
    return r


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(128, 128, 32), (1, 1, 1), (300, 257, 77), (64, 1536, 512),
                                   (513, 16, 512), (130, 200, 4096), (7, 9, 0),
                                   (300, 260, 84), (129, 516, 36)])  # partial tiles and k-tails, N % 4 == 0
def test_gemm_variants(orc, g, ta, tb, M, N, K):
    rng = np.random.default_rng(M * 7 + N * 3 + K + 10 * ta + tb)
    a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    c = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    print(f"[gemm] ta={ta} tb={tb} M={M} N={N} K={K}", flush=True)
    got = g.gemm(a, b, trans_a=bool(ta), trans_b=bool(tb))
    assert orc.rel_err(got, _ref_gemm(a, b, ta, tb, 1.0, 0.0, None, None)) <= FWD_TOL
    got = g.gemm(a, b, trans_a=bool(ta), trans_b=bool(tb), alpha=0.5, beta=1.0, c=c, bias=bias)
    assert orc.rel_err(got, _ref_gemm(a, b, ta, tb, 0.5, 1.0, c, bias)) <= FWD_TOL


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_gemm_direct_to_lds_tiles_with_edges(orc, g, ta, tb):
    # 8100 x 1020 output: 64 x 4 blocks of 128 x 256 fill one round of the
    # CUs, so the direct-to-LDS 128 x 256 tile runs, with a partial last row
    # tile, a partial last column tile and a k-tail (84 = 5 x 16 + 4)
    M, N, K = 8100, 1020, 84
    rng = np.random.default_rng(40 + 2 * ta + tb)
    a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    c = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    print(f"[gemm] direct-to-LDS ta={ta} tb={tb} M={M} N={N} K={K}", flush=True)
    got = g.gemm(a, b, trans_a=bool(ta), trans_b=bool(tb), alpha=0.5, beta=1.0, c=c, bias=bias)
    assert orc.rel_err(got, _ref_gemm(a, b, ta, tb, 0.5, 1.0, c, bias)) <= FWD_TOL


def test_gemm_split_k_projection_weight_grad(orc, g):
    # dW_qkv = x^T d_qkv at config[3]: 512 x 1536 output, K = 16384 tokens
    rng = np.random.default_rng(11)
    x = rng.standard_normal((16384, 512)).astype(np.float32)
    d = rng.standard_normal((16384, 1536)).astype(np.float32)
    print("[gemm] split-K TN 512x1536x16384", flush=True)
    got = g.gemm(x, d, trans_a=True)
    assert orc.rel_err(got, x.astype(np.float64).T @ d.astype(np.float64)) <= FWD_TOL
    # deterministic: same bits on a rerun
    np.testing.assert_array_equal(got, g.gemm(x, d, trans_a=True))


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_gemm_split_k_direct_to_lds_with_edges(orc, g, ta, tb):
    # 500 x 1532 output, K = 16380: ten K splits of 1664 (the last 1404, a
    # k-tail of 12) over 4 x 6 tiles of 128 x 256 fill the CUs, so the split
    # products run on the direct-to-LDS tile, with partial last row and column
    # tiles, then the split-K reduction with alpha, beta, C and the bias
    M, N, K = 500, 1532, 16380
    rng = np.random.default_rng(60 + 2 * ta + tb)
    a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    c = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    print(f"[gemm] split-K direct-to-LDS ta={ta} tb={tb} M={M} N={N} K={K}", flush=True)
    got = g.gemm(a, b, trans_a=bool(ta), trans_b=bool(tb), alpha=0.5, beta=1.0, c=c, bias=bias)
    assert orc.rel_err(got, _ref_gemm(a, b, ta, tb, 0.5, 1.0, c, bias)) <= FWD_TOL
    np.testing.assert_array_equal(got, g.gemm(a, b, trans_a=bool(ta), trans_b=bool(tb), alpha=0.5, beta=1.0,
                                              c=c, bias=bias))


def _dev(a):
    from asca_amd.gpu import DevBuf

    return DevBuf.from_host(np.ascontiguousarray(a, dtype=np.float32))


@pytest.mark.parametrize("rows,cols", [(16384, 512), (16384, 1536), (70001, 1024), (1000, 37), (3, 3),
                                       (5, 2048), (33, 12)])
def test_colsum_against_float64(orc, g, rows, cols):
    # asca_colsum (the bias gradients, colsum_raw of rust/src/cuda/mod.rs:642-669)
    # over wide, ragged and tiny shapes; with accumulate the sums are added to what
    # out holds; reruns give the same bits
    from asca_amd import _lib
    from asca_amd.gpu import DevBuf, _vp

    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    base = rng.standard_normal(cols).astype(np.float32)
    print(f"[colsum] {rows}x{cols}", flush=True)
    bx = _dev(x)
    s1, s2, s3 = DevBuf(cols * 4), DevBuf.from_host(base), DevBuf(cols * 4)
    _lib.call("asca_colsum", _vp(bx), rows, cols, _vp(s1), 0, None)
    _lib.call("asca_colsum", _vp(bx), rows, cols, _vp(s2), 1, None)
    _lib.call("asca_colsum", _vp(bx), rows, cols, _vp(s3), 0, None)
    _lib.call("asca_sync")
    ref = x.astype(np.float64).sum(axis=0)
    got = s1.to_host((cols,))
    assert orc.rel_err(got, ref) <= FWD_TOL
    assert orc.rel_err(s2.to_host((cols,)), ref + base.astype(np.float64)) <= FWD_TOL
    np.testing.assert_array_equal(got, s3.to_host((cols,)))
    for b in (bx, s1, s2, s3):
        b.free()


def test_gemm_and_colsum_workspace_variants_bit_identical(g):
    # asca_gemm_ws / asca_colsum_ws (caller workspace) give the bits of
    # asca_gemm / asca_colsum (stream-ordered scratch), split and unsplit
    from asca_amd import _lib
    from asca_amd.gpu import DevBuf, _vp

    rng = np.random.default_rng(12)
    for (M, N, K) in ((512, 1536, 16384), (512, 512, 8192), (96, 80, 700)):
        x = rng.standard_normal((K, M)).astype(np.float32)
        d = rng.standard_normal((K, N)).astype(np.float32)
        bx, bd = _dev(x), _dev(d)
        wsb = C.c_size_t()
        _lib.call("asca_gemm_ws_bytes", 1, 0, M, N, K, C.byref(wsb))
        print(f"[gemm] ws variant TN {M}x{N}x{K}: workspace {wsb.value} B", flush=True)
        ws = DevBuf(max(wsb.value, 4))
        c1, c2 = DevBuf(M * N * 4), DevBuf(M * N * 4)
        _lib.call("asca_gemm", 1, 0, M, N, K, 1.0, _vp(bx), M, _vp(bd), N, 0.0, _vp(c1), N, None, None)
        _lib.call("asca_gemm_ws", 1, 0, M, N, K, 1.0, _vp(bx), M, _vp(bd), N, 0.0, _vp(c2), N, None, _vp(ws),
                  wsb.value, None)
        s1, s2 = DevBuf(N * 4), DevBuf(N * 4)
        _lib.call("asca_colsum_ws_bytes", K, N, C.byref(wsb))
        ws2 = DevBuf(max(wsb.value, 4))
        _lib.call("asca_colsum", _vp(bd), K, N, _vp(s1), 0, None)
        _lib.call("asca_colsum_ws", _vp(bd), K, N, _vp(s2), 0, _vp(ws2), wsb.value, None)
        _lib.call("asca_sync")
        np.testing.assert_array_equal(c1.to_host((M, N)), c2.to_host((M, N)))
        np.testing.assert_array_equal(s1.to_host((N,)), s2.to_host((N,)))
        for b in (bx, bd, ws, c1, c2, s1, s2, ws2):
            b.free()
    # a workspace declared smaller than asked for is refused (every buffer is
    # allocated at full size, so nothing could go out of bounds either way)
    from asca_amd._lib import AscaError

    M, N, K = 512, 512, 8192
    _lib.call("asca_gemm_ws_bytes", 1, 0, M, N, K, C.byref(wsb))
    assert wsb.value > 16
    bx, bd, c, ws = DevBuf(K * M * 4), DevBuf(K * N * 4), DevBuf(M * N * 4), DevBuf(wsb.value)
    with pytest.raises(AscaError) as ei:
        _lib.call("asca_gemm_ws", 1, 0, M, N, K, 1.0, _vp(bx), M, _vp(bd), N, 0.0, _vp(c), N, None, _vp(ws), 16,
                  None)
    assert ei.value.code == 1
    _lib.call("asca_sync")
    for b in (bx, bd, c, ws):
        b.free()


def test_split_k_gemms_and_colsums_on_two_streams_concurrently(g):
    # Split-K products and column sums queued on two streams at once, next to a
    # model backward on a third, give the bits of the same calls run one after
    # another: no scratch is shared between streams.
    from asca_amd import _lib
    from asca_amd.gpu import DevBuf, _vp
    from asca_amd.model import DeviceModel
    from oracle import model_oracle as mo

    rng = np.random.default_rng(13)
    shapes = [(512, 1536, 16384), (512, 512, 16384), (256, 768, 8192), (512, 1536, 12288)]
    ins = []
    for (M, N, K) in shapes:
        ins.append((_dev(rng.standard_normal((K, M))), _dev(rng.standard_normal((K, N)))))
    def run(streams):
        outs = []
        for i, ((M, N, K), (bx, bd)) in enumerate(zip(shapes, ins)):
            st = streams[i % len(streams)]
            c, s = DevBuf(M * N * 4), DevBuf(N * 4)
            _lib.call("asca_gemm", 1, 0, M, N, K, 1.0, _vp(bx), M, _vp(bd), N, 0.0, _vp(c), N, None, st)
            _lib.call("asca_colsum", _vp(bd), K, N, _vp(s), 0, st)
            outs.append((c, s))
        return outs

    seq = run([None])
    _lib.call("asca_sync")
    ref = [(c.to_host((M, N)), s.to_host((N,))) for (c, s), (M, N, K) in zip(seq, shapes)]
    cfg = (256, 512, 8, 2, 16, 1024)
    dm = DeviceModel(*cfg)
    dm.set_params(mo.init_params(3, *cfg))
    ids = rng.integers(0, 256, 2 * 512).astype(np.uint32)
    tgts = rng.integers(0, 256, 2 * 512).astype(np.uint32)
    st = [C.c_void_p(), C.c_void_p(), C.c_void_p()]
    for x in st:
        _lib.call("asca_stream_create", C.byref(x))
    bi, bt = dm.upload_batch(ids, tgts)
    for rep in range(2):
        print(f"[gemm] two streams + model backward, repetition {rep}", flush=True)
        dm.forward_backward_dev(bi, bt, 2, 512, sync=False, stream=st[2])
        par = run([st[0], st[1]])
        _lib.call("asca_sync")
        for (c, s), (rc_, rs_), (M, N, K) in zip(par, ref, shapes):
            np.testing.assert_array_equal(c.to_host((M, N)), rc_)
            np.testing.assert_array_equal(s.to_host((N,)), rs_)
            c.free()
            s.free()
    for x in st:
        _lib.call("asca_stream_destroy", x)
    dm.close()


def test_gemm_unaligned_leading_dimensions(orc, g):
    from asca_amd import _lib
    from asca_amd.gpu import DevBuf, _vp

    rng = np.random.default_rng(5)
    M, N, K, lda, ldb, ldc = 70, 45, 33, 35, 47, 49  # odd strides: scalar load path
    a = rng.standard_normal((M, lda)).astype(np.float32)
    b = rng.standard_normal((K, ldb)).astype(np.float32)
    c = np.zeros((M, ldc), dtype=np.float32)
    ba, bb, bc = DevBuf.from_host(a), DevBuf.from_host(b), DevBuf.from_host(c)
    _lib.call("asca_gemm", 0, 0, M, N, K, 1.0, _vp(ba), lda, _vp(bb), ldb, 0.0, _vp(bc), ldc, None, None)
    _lib.call("asca_sync")
    out = bc.to_host((M, ldc))
    ref = a[:, :K].astype(np.float64) @ b[:, :N].astype(np.float64)
    assert orc.rel_err(out[:, :N], ref) <= FWD_TOL
    np.testing.assert_array_equal(out[:, N:], 0.0)  # nothing written past N


@pytest.mark.parametrize("rows,cols", [(16384, 512), (1000, 37), (3, 3), (5, 2048)])
def test_rmsnorm_fwd_bwd(orc, g, rows, cols):
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    dy = rng.standard_normal((rows, cols)).astype(np.float32)
    print(f"[rmsnorm] {rows}x{cols}", flush=True)
    y, inv = g.rmsnorm(x, 1e-6)
    assert orc.rel_err(y, orc.rmsnorm(x)) <= FWD_TOL
    ref_inv = 1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1) + 1e-6)
    assert orc.rel_err(inv, ref_inv) <= FWD_TOL
    assert orc.rel_err(g.rmsnorm_bwd(x, dy, 1e-6), orc.rmsnorm_bwd(x, dy)) <= GRAD_TOL


@pytest.mark.parametrize("n,E", [(16384, 16), (1, 1), (1000, 64), (0, 16), (70001, 7), (256, 16)])
def test_hash_route_bit_exact(orc, g, n, E):
    rng = np.random.default_rng(n + E)
    ids = rng.integers(0, 256, n).astype(np.uint32) if n != 256 else np.arange(256, dtype=np.uint32)
    print(f"[route] n={n} E={E}", flush=True)
    expert, perm, off = g.hash_route(ids, E)
    ref = orc.hash_route(ids, E)
    np.testing.assert_array_equal(expert, ref)
    rperm, roff = orc.buckets(ref, E) if n else (np.zeros(0, np.int32), np.zeros(E + 1, np.int32))
    np.testing.assert_array_equal(off, roff)
    np.testing.assert_array_equal(perm, rperm)
    if n == 256 and E == 16:
        # per-expert id counts over 0..255 (fixture computed from model.rs:70-77)
        np.testing.assert_array_equal(np.diff(off), [14, 20, 19, 17, 14, 18, 18, 20, 15, 15, 12, 19, 15, 13, 10, 17])


@pytest.mark.parametrize("E", [2, 8, 16])
def test_hash_route_replays_golden_ids(g, E):
    """Token ids 0..4095 (beyond the byte vocabulary) against the golden
    expert ids of hash_expert (rust/src/model.rs:70-77) in tests/golden."""
    import json

    from conftest import GOLDEN

    gold = np.array(json.loads((GOLDEN / "hash.json").read_text())[str(E)], dtype=np.int32)
    expert, perm, off = g.hash_route(np.arange(4096, dtype=np.uint32), E)
    np.testing.assert_array_equal(expert, gold)
    np.testing.assert_array_equal(np.diff(off), np.bincount(gold, minlength=E))
    # counting-sort order: experts ascending, token order kept within an expert
    np.testing.assert_array_equal(perm, np.argsort(gold, kind="stable"))


@pytest.mark.parametrize("E", [16, 7, 256])
def test_hash_route_full_range_ids(orc, g, E):
    """Random ids over the whole u32 range, the top bits included."""
    rng = np.random.default_rng(E)
    ids = rng.integers(0, 2 ** 32, 100000, dtype=np.uint64).astype(np.uint32)
    ids[:4] = [0, 1, 2 ** 31, 2 ** 32 - 1]
    expert, perm, off = g.hash_route(ids, E)
    ref = orc.hash_route(ids, E)
    np.testing.assert_array_equal(expert, ref)
    rperm, roff = orc.buckets(ref, E)
    np.testing.assert_array_equal(off, roff)
    np.testing.assert_array_equal(perm, rperm)


@pytest.mark.parametrize("cols", [512, 37])
def test_gather_scatter_bit_exact(g, cols):
    rng = np.random.default_rng(cols)
    src = rng.standard_normal((1000, cols)).astype(np.float32)
    idx = rng.permutation(1000)[:640].astype(np.int32)
    np.testing.assert_array_equal(g.gather_rows(src, idx), src[idx])
    dst = rng.standard_normal((1000, cols)).astype(np.float32)
    ref = dst.copy()
    ref[idx] = src[:640]
    g.scatter_rows(src[:640], idx, dst)
    np.testing.assert_array_equal(dst, ref)


@pytest.mark.parametrize("T,V", [(16384, 256), (37, 1000), (1, 5)])
def test_cross_entropy(orc, g, T, V):
    rng = np.random.default_rng(T + V)
    logits = (2 * rng.standard_normal((T, V))).astype(np.float32)
    targets = rng.integers(0, V, T).astype(np.uint32)
    print(f"[ce] T={T} V={V}", flush=True)
    loss, dl = g.cross_entropy_bwd(logits, targets)
    rloss, rdl = orc.cross_entropy(logits, targets)
    assert abs(loss - rloss) <= FWD_TOL * max(1.0, abs(rloss))
    assert orc.rel_err(dl, rdl) <= GRAD_TOL


@pytest.mark.parametrize("T,d,V", [(16384, 512, 256),   # configs[3]'s head
                                   (512, 192, 12288),   # the reference's head gate (rust/src/main.rs:1058-1097)
                                   (37, 20, 1000)])
def test_head_resident(orc, g, T, d, V):
    """head_forward_dev + head_bwd_dev (rust/src/cuda/mod.rs:826-908): the
    logits stay on the device; loss, d_head and dh match the CPU path, and
    the device path gives what the host path (logits downloaded, CE, two
    GEMMs) gives on the same GPU, bit for bit where it runs the same kernels."""
    rng = np.random.default_rng(T + d + V)
    h = rng.uniform(-0.5, 0.5, (T, d)).astype(np.float32)
    head = rng.uniform(-0.05, 0.05, (d, V)).astype(np.float32)
    targets = rng.integers(0, V, T).astype(np.uint32)
    print(f"[head] T={T} d={d} V={V}", flush=True)
    dev = g.head_forward_dev(h, head)
    try:
        logits = dev.to_host()
        loss, d_head, dh = g.head_bwd_dev(dev, targets, np.ascontiguousarray(head.T))
    finally:
        dev.free()
    ref_logits = (h.astype(np.float64) @ head.astype(np.float64)).astype(np.float32)
    assert orc.rel_err(logits, ref_logits) <= FWD_TOL
    rloss, rdl = orc.cross_entropy(ref_logits, targets)
    assert abs(loss - rloss) <= FWD_TOL * max(1.0, abs(rloss))
    assert orc.rel_err(d_head, h.astype(np.float64).T @ rdl.astype(np.float64)) <= GRAD_TOL
    assert orc.rel_err(dh, rdl.astype(np.float64) @ head.astype(np.float64).T) <= GRAD_TOL
    # host path on the same logits: same CE kernel, same d_head GEMM
    hloss, hdl = g.cross_entropy_bwd(logits, targets)
    assert loss == hloss
    np.testing.assert_array_equal(d_head, g.matmul_ta(h, hdl))
    assert orc.rel_err(dh, g.matmul_t(hdl, head)) <= GRAD_TOL


def test_head_bwd_dev_rejects_bad_shapes(g):
    h = np.zeros((8, 4), np.float32)
    dev = g.head_forward_dev(h, np.zeros((4, 6), np.float32))
    try:
        with pytest.raises(ValueError):
            g.head_bwd_dev(dev, np.zeros(7, np.uint32), np.zeros((6, 4), np.float32))
        with pytest.raises(ValueError):
            g.head_bwd_dev(dev, np.zeros(8, np.uint32), np.zeros((4, 6), np.float32))
    finally:
        dev.free()
    with pytest.raises(ValueError):
        g.head_forward_dev(h, np.zeros((5, 6), np.float32))


def test_adamw_bit_exact_over_steps(orc, g):
    rng = np.random.default_rng(9)
    n = 100003
    p = (0.02 * rng.standard_normal(n)).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    pr, mr, vr = p.copy(), m.copy(), v.copy()
    step = 0
    for s in range(1, 4):
        grad = rng.standard_normal(n).astype(np.float32)
        lr, eps_t, wd = g.adamw_scalars(3e-4, 0.9, 0.95, 1e-8, 0.01, s)
        g.adamw_update(p, grad, m, v, lr, 0.9, 0.95, eps_t, wd)
        step = orc.adamw(pr, grad, mr, vr, 3e-4, step)
        np.testing.assert_array_equal(p, pr)
        np.testing.assert_array_equal(m, mr)
        np.testing.assert_array_equal(v, vr)


def _moe_inputs(seed, T, d, d_ff, E):
    rng = np.random.default_rng(seed)
    xn = rng.standard_normal((T, d)).astype(np.float32)
    w1 = (rng.standard_normal((d, E * d_ff)) / np.sqrt(d)).astype(np.float32)
    b1 = (0.1 * rng.standard_normal(E * d_ff)).astype(np.float32)
    w2 = (rng.standard_normal((E * d_ff, d)) / np.sqrt(d_ff)).astype(np.float32)
    b2 = (0.1 * rng.standard_normal(d)).astype(np.float32)
    ids = rng.integers(0, 256, T).astype(np.uint32)
    dout = rng.standard_normal((T, d)).astype(np.float32)
    return xn, w1, b1, w2, b2, ids, dout


def _buckets(orc, ids, E):
    route = orc.hash_route(ids, E)
    perm, off = orc.buckets(route, E)
    return route, perm, [perm[off[e]:off[e + 1]].tolist() for e in range(E)]


@pytest.mark.parametrize("T,d,d_ff,E", [(1024, 256, 512, 16), (300, 64, 96, 5), (9, 8, 8, 16),
                                        (200, 30, 50, 3), (150, 32, 64, 1)])
def test_moe_fwd_bwd(orc, g, T, d, d_ff, E):
    xn, w1, b1, w2, b2, ids, dout = _moe_inputs(T + d, T, d, d_ff, E)
    route, perm, buckets = _buckets(orc, ids, E)
    print(f"[moe] T={T} d={d} d_ff={d_ff} E={E}", flush=True)
    out, dev = g.moe_forward_dev(xn, w1, b1, w2, b2, buckets, d_ff)
    r_out, r_pre, r_hid = orc.moe_fwd(xn, w1, b1, w2, b2, route, d_ff)
    assert orc.rel_err(out, r_out) <= FWD_TOL
    pe, he = dev.download_pre_hidden()
    assert orc.rel_err(np.concatenate(pe), r_pre[perm]) <= FWD_TOL
    assert orc.rel_err(np.concatenate(he), r_hid[perm]) <= FWD_TOL
    bw = g.moe_bwd_dev(dev, dout)
    ref = orc.moe_bwd(xn, w1, w2, r_pre, r_hid, route, dout, d_ff)
    for name, got, want in zip(("dxn", "dw1", "db1", "dw2", "db2"),
                               (bw.dxn, bw.d_w1, bw.d_b1, bw.d_w2, bw.d_b2), ref):
        err = orc.rel_err(got, want)
        print(f"[moe]   {name} rel err {err:.2e}", flush=True)
        assert err <= GRAD_TOL, name


def test_moe_config3_shape_by_token_subsets(orc, g):
    """configs[3] MoE (T=16384, d=512, d_ff=1024, E=16, ids U{0..255}) at full
    size.  Each token's output depends only on its own row, and with dout zero
    outside a token subset every gradient equals the subset's own gradient, so
    the oracle runs on 96 tokens only."""
    T, d, d_ff, E = 16384, 512, 1024, 16
    xn, w1, b1, w2, b2, ids, dout = _moe_inputs(2, T, d, d_ff, E)
    route, perm, buckets = _buckets(orc, ids, E)
    sub = np.sort(np.random.default_rng(0).choice(T, 96, replace=False))
    print("[moe] configs[3] full shape", flush=True)
    out, dev = g.moe_forward_dev(xn, w1, b1, w2, b2, buckets, d_ff)
    xs = np.ascontiguousarray(xn[sub])
    rs = np.ascontiguousarray(route[sub])
    r_out, r_pre, r_hid = orc.moe_fwd(xs, w1, b1, w2, b2, rs, d_ff)
    assert orc.rel_err(out[sub], r_out) <= FWD_TOL
    dmask = np.zeros_like(dout)
    dmask[sub] = dout[sub]
    bw = g.moe_bwd_dev(dev, dmask)
    ref = orc.moe_bwd(xs, w1, w2, r_pre, r_hid, rs, np.ascontiguousarray(dout[sub]), d_ff)
    dxn_ref = np.zeros_like(dout)
    dxn_ref[sub] = ref[0]
    for name, got, want in zip(("dxn", "dw1", "db1", "dw2", "db2"),
                               (bw.dxn, bw.d_w1, bw.d_b1, bw.d_w2, bw.d_b2), (dxn_ref, *ref[1:])):
        err = orc.rel_err(got, want)
        print(f"[moe]   {name} rel err {err:.2e}", flush=True)
        assert err <= GRAD_TOL, name
