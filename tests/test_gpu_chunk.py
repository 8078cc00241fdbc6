"""GPU parity of the chunked (WY/UT) form (asca_chunk_fwd / asca_chunk_bwd)
against the recurrent CPU oracle (the reference's scan_cpu / bptt_cpu
restatement) on the same bf16-rounded inputs, as configs[2] prescribes.

Bars: forward <= 2e-5 and every raw gradient <= 1e-4 as max|gpu-cpu|/max|cpu|
(rust/src/main.rs:1021-1029).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FWD_TOL = 2e-5
GRAD_TOL = 1e-4


def _extreme_gates(x, B, T):
    # the gate patterns of test_gpu_delta.test_extreme_gates: exact zeros and
    # 1e-6, a stretch of 0.005 (running products underflow), ones and 1.5
    t = np.arange(B * T) % T
    a = x.alpha.reshape(B * T, -1)
    a[(t >= 16) & (t < 32)] = 0.005
    a[(t >= 40) & (t < 44), 0] = 1.0
    a[(t >= 44) & (t < 48)] = 1.5
    a[t % 37 == 5] = 0.0
    a[t % 11 == 3, -1] = 1e-6


def _check(orc, g, seed, B, T, H, dh, C, tag, gates=None):
    from asca_amd.gpu import from_bf16, to_bf16

    print(f"[chunk] {tag} B={B} T={T} H={H} dh={dh} C={C}", flush=True)
    x = orc.DeltaInputs(seed, B, T, H, dh)
    if gates is not None:
        gates(x, B, T)
    qb, kb, vb, db_ = (to_bf16(a) for a in (x.q, x.k, x.v, x.d_o))
    q, k, v, d_o = (np.ascontiguousarray(from_bf16(a)) for a in (qb, kb, vb, db_))
    o_ref, dq, dk, dv, da, dbt = orc.delta_fwd_bwd(q, k, v, x.alpha, x.beta, d_o, B, T, H, dh)
    o, dev = g.delta_chunked(qb, kb, vb, x.alpha, x.beta, B, T, H, dh, C)
    errs = {"o": orc.rel_err(o, o_ref)}
    got = g.delta_chunked_bwd(dev, db_)
    for name, a, ref in zip(("dq", "dk", "dv", "dalpha", "dbeta"), got, (dq, dk, dv, da, dbt)):
        errs[name] = orc.rel_err(a, ref)
    print(f"[chunk] {tag} rel errors " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert errs["o"] <= FWD_TOL, errs
    for kk in errs:
        assert errs[kk] <= GRAD_TOL, (kk, errs)


@pytest.mark.parametrize("B,T,H,dh,C", [
    (4, 128, 4, 32, 64),    # configs[0] shape
    (2, 100, 2, 64, 64),    # ragged last chunk
    (2, 70, 3, 16, 16),     # small chunks
    (1, 256, 2, 128, 64),   # configs[2] head size
    (1, 5, 1, 8, 64),       # one short chunk
    (2, 96, 2, 128, 32),
    (2, 200, 2, 128, 64),   # fused C=64 dh=128 path, ragged last chunk (8 steps)
    (1, 37, 3, 128, 64),    # fused path, a single partial chunk
])
def test_chunked_matches_recurrent(orc, g, B, T, H, dh, C):
    _check(orc, g, 40 + T, B, T, H, dh, C, "shape")


def test_chunked_config2_full_size(orc, g):
    # B=8, T=4096, H=16, dh=128, chunk 64, bf16 inputs, seed 0
    _check(orc, g, 0, 8, 4096, 16, 128, 64, "configs[2]")


@pytest.mark.parametrize("B,T,H,dh,C", [
    (2, 150, 2, 128, 64),   # fused C = 64, dh = 128 kernels, ragged last chunk
    (2, 75, 3, 32, 16),     # decomposed path
    (1, 100, 2, 64, 64),
])
def test_chunked_extreme_gates(orc, g, B, T, H, dh, C):
    # dalpha takes every running product with alpha_m left out instead of
    # dividing by alpha_m: finite and at the bar for alpha = 0 and 1e-6
    _check(orc, g, 7 + dh, B, T, H, dh, C, "extreme gates", gates=_extreme_gates)


# -- f32 inputs (asca_chunk_fwd_f32 / asca_chunk_bwd_f32): the chunked form on
# the recurrent configs' f32 q, k, v, dO, against the same f32 oracle, with no
# bf16 rounding anywhere.

def _check_f32(orc, g, seed, B, T, H, dh, C, tag, gates=None, shift=False):
    """shift: q, k, v and dO one float past a 16-byte boundary on the device
    (the input copies then load with scalar accesses)."""
    import ctypes as Ct
    from asca_amd import _lib
    from asca_amd.gpu import DevBuf, _vp

    print(f"[chunk f32] {tag} B={B} T={T} H={H} dh={dh} C={C}", flush=True)
    x = orc.DeltaInputs(seed, B, T, H, dh)
    if gates is not None:
        gates(x, B, T)
    o_ref, dq, dk, dv, da, dbt = orc.delta_fwd_bwd(x.q, x.k, x.v, x.alpha, x.beta, x.d_o, B, T, H, dh)
    if not shift:
        o, dev = g.delta_chunked_f32(x.q, x.k, x.v, x.alpha, x.beta, B, T, H, dh, C)
        try:
            errs = {"o": orc.rel_err(o, o_ref)}
            got = g.delta_chunked_f32_bwd(dev, x.d_o)
        finally:
            dev.free()
    else:
        rows, d = B * T, H * dh
        bufs, ptr = [], {}
        for name in ("q", "k", "v", "d_o"):
            a = getattr(x, name)
            buf = DevBuf((a.size + 1) * 4)
            buf.upload(np.concatenate([np.zeros(1, np.float32), a.ravel()]))
            bufs.append(buf)
            ptr[name] = buf.ptr + 4
        al, be = DevBuf.from_host(x.alpha), DevBuf.from_host(x.beta)
        wsb = Ct.c_size_t()
        _lib.call("asca_chunk_ws_bytes_f32", B, T, H, dh, C, Ct.byref(wsb))
        ws, ob = DevBuf(wsb.value), DevBuf(rows * d * 4)
        outs = [DevBuf(rows * d * 4) for _ in range(3)] + [DevBuf(rows * H * 4) for _ in range(2)]
        try:
            _lib.call("asca_chunk_fwd_f32", _vp(ptr["q"]), _vp(ptr["k"]), _vp(ptr["v"]), _vp(al), _vp(be),
                      _vp(ob), _vp(ws), B, T, H, dh, C, None)
            _lib.call("asca_chunk_bwd_f32", _vp(ptr["d_o"]), _vp(ws), *[_vp(t) for t in outs], B, T, H, dh, C,
                      None)
            _lib.call("asca_sync")
            errs = {"o": orc.rel_err(ob.to_host((rows, d)), o_ref)}
            got = [t.to_host((rows, d)) for t in outs[:3]] + [t.to_host((rows, H)) for t in outs[3:]]
        finally:
            for b in (*bufs, al, be, ws, ob, *outs):
                b.free()
    for name, a, ref in zip(("dq", "dk", "dv", "dalpha", "dbeta"), got, (dq, dk, dv, da, dbt)):
        errs[name] = orc.rel_err(a, ref)
    print(f"[chunk f32] {tag} rel errors " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert errs["o"] <= FWD_TOL, errs
    for kk in errs:
        assert errs[kk] <= GRAD_TOL, (kk, errs)


@pytest.mark.parametrize("C", [16, 32, 64])
def test_chunked_f32_config1_full_size(orc, g, C):
    # B=32, T=512, H=8, dh=64, f32, seed 1 -- the headline shape
    _check_f32(orc, g, 1, 32, 512, 8, 64, C, "configs[1]")


@pytest.mark.parametrize("B,T,H,dh,C", [
    (4, 128, 4, 32, 64),    # configs[0] shape
    (2, 100, 2, 64, 32),    # ragged last chunk
    (1, 5, 1, 8, 64),       # one short chunk
    (2, 200, 2, 128, 64),   # C = 64, dh = 128 on the batched path, not the bf16 fused kernels
])
def test_chunked_f32_shapes(orc, g, B, T, H, dh, C):
    _check_f32(orc, g, 60 + T, B, T, H, dh, C, "shape")


def test_chunked_f32_unaligned_inputs(orc, g):
    _check_f32(orc, g, 3, 2, 64, 2, 64, 32, "unaligned", shift=True)


@pytest.mark.parametrize("B,T,H,dh,C", [(2, 150, 2, 64, 32), (1, 100, 2, 64, 64)])
def test_chunked_f32_extreme_gates(orc, g, B, T, H, dh, C):
    _check_f32(orc, g, 9 + dh, B, T, H, dh, C, "extreme gates", gates=_extreme_gates)
