"""ctypes wrapper of the C oracle (oracle/oracle.c) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the checker / the timed CPU baseline.  The product package
(asca_amd/) never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"

_f = np.float32
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        vp, i, l, fl, u64 = C.c_void_p, C.c_int, C.c_long, C.c_float, C.c_uint64
        sig = {
            "orc_has_avx2": (i, []),
            "orc_sdot": (fl, [vp, vp, i]),
            "orc_rng_u64": (None, [u64, vp, i]),
            "orc_rng_normal": (None, [u64, vp, l]),
            "orc_l2norm_heads": (None, [vp, vp, l, i, i]),
            "orc_delta_inputs": (None, [u64, i, i, i, i, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
            "orc_delta_scan": (None, [vp, vp, vp, vp, vp, i, i, i, i, vp, vp]),
            "orc_delta_bptt_raw": (None, [vp] * 7 + [i, i, i, i] + [vp] * 5),
            "orc_norm_backward": (None, [vp, vp, vp, l, i, i]),
            "orc_delta_fuse_grads": (None, [vp] * 11 + [l, i, i, vp, vp]),
            "orc_delta_fwd_bwd_unitwise": (None, [vp] * 6 + [i, i, i, i, i] + [vp] * 6),
            "orc_delta_decode_step": (None, [vp, vp, vp, vp, i, i, i]),
            "orc_rmsnorm": (None, [vp, vp, l, i, fl]),
            "orc_rmsnorm_bwd": (None, [vp, vp, vp, l, i, fl]),
            "orc_hash_route": (None, [vp, l, i, vp]),
            "orc_adamw": (None, [vp, vp, vp, vp, l, fl, fl, fl, fl, fl, vp]),
            "orc_moe_fwd": (None, [vp] * 6 + [l, i, i, i] + [vp] * 3),
            "orc_moe_bwd": (None, [vp] * 7 + [l, i, i, i] + [vp] * 5),
            "orc_cross_entropy": (fl, [vp, vp, l, i, vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


def _z(*shape):
    return np.zeros(shape, dtype=_f)


# ------------------------------------------------------------------ rng


def rng_u64(seed: int, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.uint64)
    lib().orc_rng_u64(seed, _p(out), n)
    return out


def rng_normal(seed: int, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=_f)
    lib().orc_rng_normal(seed, _p(out), n)
    return out


# ---------------------------------------------------------------- delta


class DeltaInputs:
    """Seeded inputs of a delta config: q, k (L2-normalised), v, alpha, beta,
    dO, plus the saved norms qn, kn and the raw gate logits (rows, 2H)."""

    def __init__(self, seed: int, B: int, T: int, H: int, dh: int):
        self.seed, self.B, self.T, self.H, self.dh = seed, B, T, H, dh
        rows, d = B * T, H * dh
        self.q, self.k, self.v, self.d_o = _z(rows, d), _z(rows, d), _z(rows, d), _z(rows, d)
        self.alpha, self.beta = _z(rows, H), _z(rows, H)
        self.qn, self.kn = _z(rows, H), _z(rows, H)
        self.gate = _z(rows, 2 * H)
        lib().orc_delta_inputs(seed, B, T, H, dh, _p(self.q), _p(self.k), _p(self.v), _p(self.alpha),
                               _p(self.beta), _p(self.d_o), _p(self.qn), _p(self.kn), _p(self.gate))


def l2norm_heads(x: np.ndarray, H: int, dh: int):
    x = np.ascontiguousarray(x, dtype=_f).copy()
    n = _z(x.shape[0], H)
    lib().orc_l2norm_heads(_p(x), _p(n), x.shape[0], H, dh)
    return x, n


def delta_scan(q, k, v, alpha, beta, B, T, H, dh, with_states=True):
    """DeltaBlock::scan_cpu: returns (o, states or None); states[(h*B+b)] has
    (T+1)*dh*dh floats."""
    o = _z(B * T, H * dh)
    st = _z(H * B, (T + 1) * dh * dh) if with_states else None
    lib().orc_delta_scan(_p(q), _p(k), _p(v), _p(alpha), _p(beta), B, T, H, dh, _p(o), _p(st))
    return o, st


def delta_bptt_raw(q, k, v, alpha, beta, d_o, states, B, T, H, dh):
    rows, d = B * T, H * dh
    dq, dk, dv, da, db = _z(rows, d), _z(rows, d), _z(rows, d), _z(rows, H), _z(rows, H)
    lib().orc_delta_bptt_raw(_p(q), _p(k), _p(v), _p(alpha), _p(beta), _p(d_o), _p(states), B, T, H, dh,
                             _p(dq), _p(dk), _p(dv), _p(da), _p(db))
    return dq, dk, dv, da, db


def delta_fuse(q, k, qn, kn, alpha, beta, dq, dk, dv, da, db, H, dh):
    rows, d = q.shape[0], H * dh
    dq, dk = dq.copy(), dk.copy()
    d_qkv, d_gate = _z(rows, 3 * d), _z(rows, 2 * H)
    lib().orc_delta_fuse_grads(_p(q), _p(k), _p(qn), _p(kn), _p(alpha), _p(beta), _p(dq), _p(dk), _p(dv),
                               _p(da), _p(db), rows, H, dh, _p(d_qkv), _p(d_gate))
    return d_qkv, d_gate


def delta_fwd_bwd(q, k, v, alpha, beta, d_o, B, T, H, dh, nthreads=None):
    """Unit-wise forward + raw BPTT (same per-unit arithmetic as the
    reference-threaded drivers, without the global history)."""
    rows, d = B * T, H * dh
    o, dq, dk, dv = _z(rows, d), _z(rows, d), _z(rows, d), _z(rows, d)
    da, db = _z(rows, H), _z(rows, H)
    nt = nthreads or min(os.cpu_count() or 1, 16)
    lib().orc_delta_fwd_bwd_unitwise(_p(q), _p(k), _p(v), _p(alpha), _p(beta), _p(d_o), B, T, H, dh, nt,
                                     _p(o), _p(dq), _p(dk), _p(dv), _p(da), _p(db))
    return o, dq, dk, dv, da, db


def delta_decode_step(states, qkv, gate, H, dh):
    n = qkv.shape[0]
    o = _z(n, H * dh)
    lib().orc_delta_decode_step(_p(states), _p(qkv), _p(gate), _p(o), n, H, dh)
    return o


def rmsnorm(x, eps=1e-6):
    y = np.zeros_like(x)
    lib().orc_rmsnorm(_p(x), _p(y), x.shape[0], x.shape[1], eps)
    return y


def rmsnorm_bwd(x, dy, eps=1e-6):
    dx = np.zeros_like(x)
    lib().orc_rmsnorm_bwd(_p(x), _p(dy), _p(dx), x.shape[0], x.shape[1], eps)
    return dx


def hash_route(ids: np.ndarray, n_experts: int) -> np.ndarray:
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    out = np.zeros(ids.shape[0], dtype=np.int32)
    lib().orc_hash_route(_p(ids), ids.shape[0], n_experts, _p(out))
    return out


def adamw(p, g, m, v, lr, step, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.01):
    """One AdamW::update on float32 arrays in place; returns the new step."""
    st = np.array([step], dtype=np.uint32)
    lib().orc_adamw(_p(p), _p(g), _p(m), _p(v), p.size, lr, beta1, beta2, eps, wd, _p(st))
    return int(st[0])


def buckets(route: np.ndarray, n_experts: int):
    """perm (tokens sorted by expert, ascending inside an expert) and CSR
    offsets, the buckets of HashMoe::forward (rust/src/model.rs:190-193)."""
    route = np.asarray(route, dtype=np.int64)
    perm = np.concatenate([np.nonzero(route == e)[0] for e in range(n_experts)]).astype(np.int32)
    counts = np.bincount(route, minlength=n_experts)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    return perm, offsets


def moe_fwd(xn, w1, b1, w2, b2, route, d_ff):
    """HashMoe::forward CPU path on normalised input; (out, pre, hidden) in
    token order."""
    T, d = xn.shape
    E = w1.shape[1] // d_ff
    route = np.ascontiguousarray(route, dtype=np.int32)
    out, pre, hidden = _z(T, d), _z(T, d_ff), _z(T, d_ff)
    lib().orc_moe_fwd(_p(xn), _p(w1), _p(b1), _p(w2), _p(b2), _p(route), T, d, d_ff, E,
                      _p(out), _p(pre), _p(hidden))
    return out, pre, hidden


def moe_bwd(xn, w1, w2, pre, hidden, route, dout, d_ff):
    """HashMoe::backward CPU path before its RMSNorm backward;
    (dxn, dw1, db1, dw2, db2) with pre/hidden in token order."""
    T, d = xn.shape
    E = w1.shape[1] // d_ff
    route = np.ascontiguousarray(route, dtype=np.int32)
    dxn, dw1, db1 = _z(T, d), _z(d, E * d_ff), _z(E * d_ff)
    dw2, db2 = _z(E * d_ff, d), _z(d)
    lib().orc_moe_bwd(_p(xn), _p(w1), _p(w2), _p(pre), _p(hidden), _p(route), _p(dout), T, d, d_ff, E,
                      _p(dxn), _p(dw1), _p(db1), _p(dw2), _p(db2))
    return dxn, dw1, db1, dw2, db2


def cross_entropy(logits, targets):
    """cpu_cross_entropy: (mean loss, dlogits)."""
    T, V = logits.shape
    t = np.ascontiguousarray(targets, dtype=np.uint32)
    dl = _z(T, V)
    loss = lib().orc_cross_entropy(_p(logits), _p(t), T, V, _p(dl))
    return float(loss), dl


def rel_err(a: np.ndarray, ref: np.ndarray) -> float:
    """max|a - ref| / max|ref|, the reference's parity metric
    (rust/src/main.rs:1021-1029)."""
    a = np.asarray(a, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = max(float(np.max(np.abs(ref))) if ref.size else 0.0, 1e-30)
    return float(np.max(np.abs(a - ref))) / scale if ref.size else 0.0
