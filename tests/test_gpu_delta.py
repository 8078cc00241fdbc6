"""GPU parity of the recurrent delta rule (forward + BPTT) against the CPU oracle.

Bars (from the north star): forward <= 2e-5 and every gradient <= 1e-4, both as
max|gpu - cpu| / max|cpu| per tensor (rust/src/main.rs:1021-1029).  Batch
isolation is bit-exact, as the reference's gate demands (main.rs:954-981).
All calls go through the C ABI (asca_amd.gpu -> libasca_hip.so).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FWD_TOL = 2e-5
GRAD_TOL = 1e-4


def _check_all(orc, g, x, B, T, H, dh, tag):
    print(f"[delta parity] {tag} B={B} T={T} H={H} dh={dh}", flush=True)
    o_ref, dq, dk, dv, da, db = orc.delta_fwd_bwd(x.q, x.k, x.v, x.alpha, x.beta, x.d_o, B, T, H, dh)
    o, dev = g.delta_scan(x.q, x.k, x.v, x.alpha, x.beta, B, T, H, dh)
    errs = {"o": orc.rel_err(o, o_ref)}
    raw = g.delta_bwd_raw(dev, x.d_o)
    for name, got, ref in zip(("dq", "dk", "dv", "dalpha", "dbeta"), raw, (dq, dk, dv, da, db)):
        errs[name] = orc.rel_err(got, ref)
    d_qkv_ref, d_gate_ref = orc.delta_fuse(x.q, x.k, x.qn, x.kn, x.alpha, x.beta, dq, dk, dv, da, db, H, dh)
    d_qkv, d_gate = g.delta_bwd_dev(dev, x.d_o, x.qn, x.kn)
    errs["d_qkv"] = orc.rel_err(d_qkv, d_qkv_ref)
    errs["d_gate"] = orc.rel_err(d_gate, d_gate_ref)
    print(f"[delta parity] {tag} rel errors " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert errs["o"] <= FWD_TOL, errs
    for k in errs:
        assert errs[k] <= GRAD_TOL, (k, errs)
    return dev


def test_wave_primitives_lane_semantics(g):
    import ctypes as C
    from asca_amd import _lib

    out = np.zeros((16, 64), dtype=np.float32)  # rows 10-13: MFMA probe (test_gpu_ops)
    _lib.call("asca_selftest_wave", out.ctypes.data_as(C.c_void_p))
    lane = np.arange(64)
    np.testing.assert_array_equal(out[0], lane ^ 1)
    np.testing.assert_array_equal(out[1], lane ^ 2)
    np.testing.assert_array_equal(out[2], (lane & ~7) | (7 - (lane & 7)))
    np.testing.assert_array_equal(out[3], (lane & ~15) | (15 - (lane & 15)))
    np.testing.assert_array_equal(out[4], lane ^ 8)
    # permlane32_swap(x, y): vdst keeps its low half and takes y's low half up top;
    # vsrc takes x's high half in its low half and keeps its own high half.
    np.testing.assert_array_equal(out[5], np.where(lane < 32, lane, 100 + lane - 32))
    np.testing.assert_array_equal(out[6], np.where(lane < 32, lane + 32, 100 + lane))
    # permlane16_swap: the same between even and odd 16-lane rows
    odd = (lane >> 4) & 1
    np.testing.assert_array_equal(out[7], np.where(odd == 0, lane, 100 + lane - 16))
    np.testing.assert_array_equal(out[8], np.where(odd == 0, lane + 16, 100 + lane))
    np.testing.assert_array_equal(out[9], np.full(64, 2016.0))
    # row_shr prefix products of z = 2^e: the first n lanes of each 16-lane row
    # hold the product of the row's lanes up to their own
    e = (lane * 3) % 5 - 2
    for row, n in ((14, 8), (15, 2)):
        pos = lane & 15
        want = np.array([2.0 ** e[l - min(pos[l], n - 1): l + 1].sum() for l in lane])
        sel = pos < n
        np.testing.assert_array_equal(out[row][sel], want[sel])


def test_config0_b4_t128_h4_dh32(orc, g):
    B, T, H, dh = 4, 128, 4, 32
    _check_all(orc, g, orc.DeltaInputs(0, B, T, H, dh), B, T, H, dh, "configs[0] seed 0")


def test_config1_b32_t512_h8_dh64(orc, g):
    B, T, H, dh = 32, 512, 8, 64
    _check_all(orc, g, orc.DeltaInputs(1, B, T, H, dh), B, T, H, dh, "configs[1] seed 1")


@pytest.mark.parametrize("B,T,H,dh", [
    (1, 1, 1, 64),      # single step
    (2, 7, 3, 8),       # dh of rust/tests/gradcheck.rs, ragged T
    (3, 24, 4, 16),     # the reference's delta_scan gate shape (main.rs:854)
    (2, 33, 2, 24),     # masked dh, T not a multiple of the checkpoint interval
    (2, 70, 2, 48),
    (1, 45, 2, 128),
    (9, 20, 16, 128),   # 144 units: dh = 128 splits its columns at any unit count
    (9, 13, 16, 100),
    (2, 17, 6, 32),     # dh of the reference's delta-grad gate (main.rs:1106), ragged T
    (5, 64, 1, 64),
    (1, 9, 2, 5),       # odd dh
])
def test_edge_shapes(orc, g, B, T, H, dh):
    _check_all(orc, g, orc.DeltaInputs(100 + B * T + dh, B, T, H, dh), B, T, H, dh, "edge")


@pytest.mark.parametrize("B,T,H,dh", [(2, 75, 2, 16), (2, 75, 3, 32), (2, 75, 2, 64), (1, 75, 2, 128), (2, 60, 2, 48)])
def test_extreme_gates(orc, g, B, T, H, dh):
    # Inside a checkpoint segment the kernels keep the state divided by the
    # running product of alpha when every alpha of the segment lies in
    # [2^-8, 2^8], and run the plain recurrence otherwise.  Cover both, and the
    # switch between them: exact zeros and 1e-6 (plain), a stretch of 0.005
    # (scaled, products down to 4e-19), exact ones and 1.5 (scaled, growing).
    x = orc.DeltaInputs(7 + dh, B, T, H, dh)
    t = np.arange(B * T) % T
    a = x.alpha.reshape(B * T, H)
    a[(t >= 16) & (t < 32)] = 0.005
    a[(t >= 40) & (t < 44), 0] = 1.0
    a[(t >= 44) & (t < 48)] = 1.5
    a[t % 37 == 5] = 0.0
    a[t % 11 == 3, -1] = 1e-6
    _check_all(orc, g, x, B, T, H, dh, "extreme gates")


def test_states_download_matches_cpu_history(orc, g):
    # rust/src/main.rs:854-953: B=3 seq=24 H=4 dh=16, full state history compared
    B, T, H, dh = 3, 24, 4, 16
    rng = np.random.default_rng(5)
    q, _ = orc.l2norm_heads(rng.standard_normal((B * T, H * dh)).astype(np.float32), H, dh)
    k, _ = orc.l2norm_heads(rng.standard_normal((B * T, H * dh)).astype(np.float32), H, dh)
    v = (0.5 * rng.standard_normal((B * T, H * dh))).astype(np.float32)
    alpha = (0.85 + 0.1 * rng.random((B * T, H))).astype(np.float32)
    beta = (0.7 + 0.2 * rng.random((B * T, H))).astype(np.float32)
    o_ref, st_ref = orc.delta_scan(q, k, v, alpha, beta, B, T, H, dh)
    o, dev = g.delta_scan(q, k, v, alpha, beta, B, T, H, dh)
    assert orc.rel_err(o, o_ref) <= FWD_TOL
    st = np.stack(dev.download_states())
    assert st.shape == st_ref.shape
    assert orc.rel_err(st, st_ref) <= FWD_TOL


def test_batch_isolation_bit_exact_on_gpu(orc, g):
    B, T, H, dh = 3, 40, 2, 64
    x = orc.DeltaInputs(21, B, T, H, dh)
    o, dev = g.delta_scan(x.q, x.k, x.v, x.alpha, x.beta, B, T, H, dh)
    d_qkv, d_gate = g.delta_bwd_dev(dev, x.d_o, x.qn, x.kn)
    for b in range(B):
        rs = slice(b * T, (b + 1) * T)
        sub = [np.ascontiguousarray(a[rs]) for a in (x.q, x.k, x.v, x.alpha, x.beta)]
        o1, dev1 = g.delta_scan(*sub, 1, T, H, dh)
        q1, g1 = g.delta_bwd_dev(dev1, np.ascontiguousarray(x.d_o[rs]), np.ascontiguousarray(x.qn[rs]),
                                 np.ascontiguousarray(x.kn[rs]))
        np.testing.assert_array_equal(o1, o[rs])
        np.testing.assert_array_equal(q1, d_qkv[rs])
        np.testing.assert_array_equal(g1, d_gate[rs])


def test_deterministic_rerun(orc, g):
    B, T, H, dh = 4, 100, 2, 64
    x = orc.DeltaInputs(8, B, T, H, dh)
    o1, dev1 = g.delta_scan(x.q, x.k, x.v, x.alpha, x.beta, B, T, H, dh)
    o2, dev2 = g.delta_scan(x.q, x.k, x.v, x.alpha, x.beta, B, T, H, dh)
    np.testing.assert_array_equal(o1, o2)
    a = g.delta_bwd_dev(dev1, x.d_o, x.qn, x.kn)
    b = g.delta_bwd_dev(dev2, x.d_o, x.qn, x.kn)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


def test_injected_failure_is_an_error_then_recovers(orc, g):
    from asca_amd import gpu
    from asca_amd._lib import AscaError

    B, T, H, dh = 2, 16, 2, 32
    x = orc.DeltaInputs(2, B, T, H, dh)
    gpu.fail_after(0)
    with pytest.raises(AscaError) as ei:
        g.delta_scan(x.q, x.k, x.v, x.alpha, x.beta, B, T, H, dh)
    assert ei.value.code == 5
    o, _ = g.delta_scan(x.q, x.k, x.v, x.alpha, x.beta, B, T, H, dh)
    o_ref, _ = orc.delta_scan(x.q, x.k, x.v, x.alpha, x.beta, B, T, H, dh)
    assert orc.rel_err(o, o_ref) <= FWD_TOL


def test_empty_and_invalid_shapes(g):
    from asca_amd._lib import AscaError

    z = np.zeros((0, 64), dtype=np.float32)
    zg = np.zeros((0, 1), dtype=np.float32)
    o, _ = g.delta_scan(z, z, z, zg, zg, 0, 5, 1, 64)
    assert o.shape == (0, 64)
    x = np.zeros((4, 129 * 1), dtype=np.float32)
    xg = np.zeros((4, 1), dtype=np.float32)
    with pytest.raises(AscaError) as ei:
        g.delta_scan(x, x, x, xg, xg, 1, 4, 1, 129)
    assert ei.value.code == 3


# dh = 64 runs on the one-block-per-unit kernels of delta_ut64.hip at any unit
# count: 16-step blocks of the UT form on the matrix cores, the state in the
# chain waves' accumulators.  One unit, few units, more units than CUs (blocks
# queued behind a full round), ragged tails (a partial last block, one inside a
# partial group of four), a single step, fewer steps than a block, and the
# extreme gate patterns of test_extreme_gates.
@pytest.mark.parametrize("B,T,H", [(129, 1, 1), (17, 5, 8), (20, 16, 8), (17, 29, 8), (33, 67, 4), (3, 40, 48),
                                   (1, 37, 1), (2, 50, 4), (40, 20, 8)])
def test_blocked_dh64_shapes(orc, g, B, T, H):
    dh = 64
    _check_all(orc, g, orc.DeltaInputs(300 + B * T + H, B, T, H, dh), B, T, H, dh, "dh64 blocked")


def test_blocked_dh64_extreme_gates(orc, g):
    B, T, H, dh = 17, 75, 8, 64
    x = orc.DeltaInputs(77, B, T, H, dh)
    t = np.arange(B * T) % T
    a = x.alpha.reshape(B * T, H)
    a[(t >= 16) & (t < 32)] = 0.005
    a[(t >= 40) & (t < 44), 0] = 1.0
    a[(t >= 44) & (t < 48)] = 1.5
    a[t % 37 == 5] = 0.0
    a[t % 11 == 3, -1] = 1e-6
    _check_all(orc, g, x, B, T, H, dh, "dh64 blocked extreme gates")


def test_blocked_dh64_batch_isolation(orc, g):
    # 136 units together, then each sequence alone (8 units); forward and fused
    # backward agree to the bar
    B, T, H, dh = 17, 24, 8, 64
    x = orc.DeltaInputs(31, B, T, H, dh)
    o, dev = g.delta_scan(x.q, x.k, x.v, x.alpha, x.beta, B, T, H, dh)
    d_qkv, d_gate = g.delta_bwd_dev(dev, x.d_o, x.qn, x.kn)
    for b in (0, 7, 16):
        rs = slice(b * T, (b + 1) * T)
        sub = [np.ascontiguousarray(a[rs]) for a in (x.q, x.k, x.v, x.alpha, x.beta)]
        o1, dev1 = g.delta_scan(*sub, 1, T, H, dh)
        q1, g1 = g.delta_bwd_dev(dev1, np.ascontiguousarray(x.d_o[rs]), np.ascontiguousarray(x.qn[rs]),
                                 np.ascontiguousarray(x.kn[rs]))
        assert orc.rel_err(o[rs], o1) <= FWD_TOL
        assert orc.rel_err(d_qkv[rs], q1) <= GRAD_TOL
        assert orc.rel_err(d_gate[rs], g1) <= GRAD_TOL


@pytest.mark.parametrize("a", [0.5, 0.6, 0.7, 0.72, 0.75, 0.8, 0.9, 0.99])
def test_blocked_dh64_constant_gates(orc, g, a):
    # Every alpha equal: each 16-step block has gate product a^16 (down to
    # 1.5e-5 at a = 0.5) in gamma, Gamma and the decay of the carried state.
    B, T, H, dh = 17, 80, 8, 64
    x = orc.DeltaInputs(500, B, T, H, dh)
    x.alpha[:] = np.float32(a)
    _check_all(orc, g, x, B, T, H, dh, f"dh64 alpha={a}")


def test_blocked_dh64_unaligned_pointers(orc, g):
    # q, k, v and dO one float past a 16-byte boundary: the blocked kernels
    # load them with scalar accesses and give the aligned results' parity.
    import ctypes as C
    from asca_amd import _lib
    from asca_amd.gpu import DevBuf, _vp

    B, T, H, dh = 17, 21, 8, 64
    x = orc.DeltaInputs(41, B, T, H, dh)
    o_ref, dq, dk, dv, da, db = orc.delta_fwd_bwd(x.q, x.k, x.v, x.alpha, x.beta, x.d_o, B, T, H, dh)
    rows, d = B * T, H * dh

    def shifted(a):
        buf = DevBuf((a.size + 1) * 4)
        flat = np.concatenate([np.zeros(1, np.float32), a.ravel()])
        buf.upload(flat)
        return buf, buf.ptr + 4

    bufs = []
    ptr = {}
    for name in ("q", "k", "v", "d_o"):
        bf, p = shifted(getattr(x, name))
        bufs.append(bf)
        ptr[name] = p
    al, be = DevBuf.from_host(x.alpha), DevBuf.from_host(x.beta)
    wsb = C.c_size_t()
    _lib.call("asca_delta_ws_bytes", B, T, H, dh, C.byref(wsb))
    ws = DevBuf(wsb.value)
    o = DevBuf(rows * d * 4)
    outs = [DevBuf(rows * d * 4) for _ in range(3)] + [DevBuf(rows * H * 4) for _ in range(2)]
    _lib.call("asca_delta_fwd", _vp(ptr["q"]), _vp(ptr["k"]), _vp(ptr["v"]), _vp(al), _vp(be), _vp(o), _vp(ws),
              B, T, H, dh, None)
    _lib.call("asca_delta_bwd_raw", _vp(ptr["q"]), _vp(ptr["k"]), _vp(ptr["v"]), _vp(al), _vp(be),
              _vp(ptr["d_o"]), _vp(ws), *[_vp(t) for t in outs], B, T, H, dh, None)
    _lib.call("asca_sync")
    got = [o.to_host((rows, d))] + [t.to_host((rows, d)) for t in outs[:3]] + [t.to_host((rows, H)) for t in outs[3:]]
    errs = [orc.rel_err(a, r) for a, r in zip(got, (o_ref, dq, dk, dv, da, db))]
    print(f"[delta parity] dh64 unaligned rel errors {errs}", flush=True)
    assert errs[0] <= FWD_TOL and max(errs[1:]) <= GRAD_TOL, errs
    for b in [*bufs, al, be, ws, o, *outs]:
        b.free()


@pytest.mark.parametrize("shift", ["inputs", "output"])
def test_blocked_dh64_fused_unaligned(orc, g, shift):
    # The fused backward (the drop-in for Gpu::delta_bwd_dev, rust/src/cuda/mod.rs:1328-1382)
    # on rows off a 16-byte boundary: q, k, v, dO one float past it ("inputs"), or
    # the d_qkv output one float past it ("output").  Either sends the call to the
    # unaligned fused instantiation, which must give the aligned path's parity.
    # (d_qkv's row stride is 3*H*dh floats, a multiple of 4 at dh = 64 for every H,
    # so an unaligned stride cannot reach this path through the C ABI.)
    import ctypes as C
    from asca_amd import _lib
    from asca_amd.gpu import DevBuf, _vp

    B, T, H, dh = 9, 37, 4, 64
    x = orc.DeltaInputs(43, B, T, H, dh)
    o_ref, dq, dk, dv, da, db = orc.delta_fwd_bwd(x.q, x.k, x.v, x.alpha, x.beta, x.d_o, B, T, H, dh)
    d_qkv_ref, d_gate_ref = orc.delta_fuse(x.q, x.k, x.qn, x.kn, x.alpha, x.beta, dq, dk, dv, da, db, H, dh)
    rows, d = B * T, H * dh
    off = 1 if shift == "inputs" else 0

    def placed(a, k):
        buf = DevBuf((a.size + k) * 4)
        buf.upload(np.concatenate([np.zeros(k, np.float32), a.ravel()]))
        return buf, buf.ptr + 4 * k

    bufs, ptr = [], {}
    for name in ("q", "k", "v", "d_o"):
        bf, p = placed(getattr(x, name), off)
        bufs.append(bf)
        ptr[name] = p
    small = {name: DevBuf.from_host(getattr(x, name)) for name in ("alpha", "beta", "qn", "kn")}
    wsb = C.c_size_t()
    _lib.call("asca_delta_ws_bytes", B, T, H, dh, C.byref(wsb))
    ws = DevBuf(wsb.value)
    o = DevBuf(rows * d * 4)
    k_out = 1 if shift == "output" else 0
    dqkv = DevBuf((rows * 3 * d + k_out) * 4)
    dgate = DevBuf(rows * 2 * H * 4)
    _lib.call("asca_delta_fwd", _vp(ptr["q"]), _vp(ptr["k"]), _vp(ptr["v"]), _vp(small["alpha"]),
              _vp(small["beta"]), _vp(o), _vp(ws), B, T, H, dh, None)
    _lib.call("asca_delta_bwd_fused", _vp(ptr["q"]), _vp(ptr["k"]), _vp(ptr["v"]), _vp(small["alpha"]),
              _vp(small["beta"]), _vp(small["qn"]), _vp(small["kn"]), _vp(ptr["d_o"]), _vp(ws),
              _vp(dqkv.ptr + 4 * k_out), _vp(dgate), B, T, H, dh, None)
    _lib.call("asca_sync")
    got_qkv = dqkv.to_host((rows * 3 * d + k_out,))[k_out:].reshape(rows, 3 * d)
    errs = {"o": orc.rel_err(o.to_host((rows, d)), o_ref),
            "d_qkv": orc.rel_err(got_qkv, d_qkv_ref),
            "d_gate": orc.rel_err(dgate.to_host((rows, 2 * H)), d_gate_ref)}
    print(f"[delta parity] dh64 fused unaligned ({shift}) rel errors {errs}", flush=True)
    assert errs["o"] <= FWD_TOL and errs["d_qkv"] <= GRAD_TOL and errs["d_gate"] <= GRAD_TOL, errs
    for b in [*bufs, *small.values(), ws, o, dqkv, dgate]:
        b.free()
