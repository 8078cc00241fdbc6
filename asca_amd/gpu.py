"""GPU backend operator API over libasca_hip, mirroring the reference's
`crate::cuda` module (rust/src/cuda/mod.rs).

Same surface, same meaning, same failure behaviour:
  * gpu() returns the process-wide Gpu or None when no usable gfx950 device
    (or no built library) is present; the reason is kept for describe()
    (mod.rs:177-237, 1488-1496, 1525-1533);
  * available / set_enabled / offload / offload_opt_in / worth_offload read
    ASCA_GPU, ASCA_GPU_OFF, ASCA_GPU_ON and ASCA_GPU_MIN once (mod.rs:1498-1596);
  * Gpu methods take host matrices (2-D float32 numpy arrays, the reference's
    `Mat`), upload, launch, synchronise and download, and raise AscaError
    (the reference's `Err(String)`) instead of aborting, so callers can fall
    back to their CPU path exactly as rust/src/delta.rs:227-240,640-647 do;
  * DevBuf is the pooled device buffer (mod.rs:100-174) and DeltaDev the
    forward->backward residency handle (mod.rs:1386-1397) -- here it holds
    state checkpoints instead of the full history, and download_states()
    rebuilds the (T+1) dh^2 history per unit by recomputation.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

import numpy as np

from . import _lib
from ._lib import AscaError

ARCH = "gfx950"
KERNELS = ("delta_fwd", "delta_bwd", "delta_states", "delta_decode")
DEFAULT_MIN_FLOPS = 4_000_000

_f32 = np.float32


def _csv_env(name: str) -> list[str]:
    v = os.environ.get(name, "")
    return [s.strip().lower() for s in v.split(",") if s.strip()]


class _Flags:
    def __init__(self):
        self.enabled = os.environ.get("ASCA_GPU") != "0"
        self.off = _csv_env("ASCA_GPU_OFF")
        self.on = _csv_env("ASCA_GPU_ON")
        try:
            self.min_flops = int(os.environ.get("ASCA_GPU_MIN", DEFAULT_MIN_FLOPS))
        except ValueError:
            self.min_flops = DEFAULT_MIN_FLOPS


_flags: _Flags | None = None
_gpu_lock = threading.Lock()
_gpu_state: dict = {"done": False, "gpu": None, "err": None}


def _f() -> _Flags:
    global _flags
    if _flags is None:
        _flags = _Flags()
    return _flags


# ----------------------------------------------------------------- buffers


class DevBuf:
    """Pooled device buffer (rust/src/cuda/mod.rs:100-174)."""

    __slots__ = ("ptr", "nbytes")

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        _lib.call("asca_alloc", C.byref(p), C.c_size_t(max(int(nbytes), 4)))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_host(cls, arr: np.ndarray) -> "DevBuf":
        a = np.ascontiguousarray(arr, dtype=_f32)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        if a.nbytes > self.nbytes:
            raise ValueError(f"upload of {a.nbytes} B into a {self.nbytes} B buffer")
        _lib.call("asca_h2d", C.c_void_p(self.ptr), a.ctypes.data_as(C.c_void_p), C.c_size_t(a.nbytes))

    def download(self, out: np.ndarray) -> np.ndarray:
        if not out.flags["C_CONTIGUOUS"]:
            raise ValueError("download target must be C-contiguous")
        if out.nbytes > self.nbytes:
            raise ValueError(f"download of {out.nbytes} B from a {self.nbytes} B buffer")
        _lib.call("asca_d2h", out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr), C.c_size_t(out.nbytes))
        return out

    def to_host(self, shape, dtype=_f32) -> np.ndarray:
        return self.download(np.empty(shape, dtype=dtype))

    def free(self) -> None:
        if self.ptr:
            try:
                _lib.call("asca_free", C.c_void_p(self.ptr))
            finally:
                self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _vp(x) -> C.c_void_p:
    if isinstance(x, DevBuf):
        return C.c_void_p(x.ptr)
    if x is None:
        return C.c_void_p(None)
    return C.c_void_p(int(x))


# ---------------------------------------------------------- residency types


class DeltaDev:
    """Delta-rule state kept on the device between forward and backward
    (rust/src/cuda/mod.rs:1386-1397).  Holds q, k, v, alpha, beta and the
    workspace of checkpoints + per-step S^T k written by the forward."""

    def __init__(self, q, k, v, alpha, beta, ws, batch, seq, n_heads, dh):
        self.q, self.k, self.v, self.alpha, self.beta, self.ws = q, k, v, alpha, beta, ws
        self.batch, self.seq, self.n_heads, self.dh = batch, seq, n_heads, dh

    def download_states(self) -> list[np.ndarray]:
        """(T+1)*dh*dh floats per unit h*B + b, S before every step then the
        final state (rust/src/cuda/mod.rs:1473-1479)."""
        B, T, H, dh = self.batch, self.seq, self.n_heads, self.dh
        per = (T + 1) * dh * dh
        buf = DevBuf(H * B * per * 4)
        try:
            _lib.call("asca_delta_states", _vp(self.q), _vp(self.k), _vp(self.v), _vp(self.alpha),
                      _vp(self.beta), _vp(buf), B, T, H, dh, None)
            _lib.call("asca_sync")
            flat = buf.to_host((H * B, per))
        finally:
            buf.free()
        return [flat[i] for i in range(H * B)]


# --------------------------------------------------------------------- Gpu


class Gpu:
    """The device handle (rust/src/cuda/mod.rs:89-95)."""

    def __init__(self, name: str, sm_count: int):
        self.name = name
        self.sm_count = sm_count

    # -- delta rule ---------------------------------------------------------
    def delta_scan(self, q, k, v, alpha, beta, batch: int, seq: int, n_heads: int, dh: int):
        """Gpu::delta_scan (rust/src/cuda/mod.rs:1253-1321): forward for all
        (head, sequence) units; returns (o, DeltaDev) with o on the host."""
        d = n_heads * dh
        t_len = batch * seq
        for name, m, cols in (("q", q, d), ("k", k, d), ("v", v, d), ("alpha", alpha, n_heads),
                              ("beta", beta, n_heads)):
            if m.shape != (t_len, cols):
                raise ValueError(f"delta_scan: {name} has shape {m.shape}, expected {(t_len, cols)}")
        wsb = C.c_size_t()
        _lib.call("asca_delta_ws_bytes", batch, seq, n_heads, dh, C.byref(wsb))
        dq, dk, dv = DevBuf.from_host(q), DevBuf.from_host(k), DevBuf.from_host(v)
        da, db = DevBuf.from_host(alpha), DevBuf.from_host(beta)
        ws = DevBuf(wsb.value)
        out = DevBuf(t_len * d * 4)
        try:
            _lib.call("asca_delta_fwd", _vp(dq), _vp(dk), _vp(dv), _vp(da), _vp(db), _vp(out), _vp(ws),
                      batch, seq, n_heads, dh, None)
            _lib.call("asca_sync")
            o = out.to_host((t_len, d))
        finally:
            out.free()
        return o, DeltaDev(dq, dk, dv, da, db, ws, batch, seq, n_heads, dh)

    def delta_bwd_dev(self, dev: DeltaDev, d_o, qnorm, knorm):
        """Gpu::delta_bwd_dev (rust/src/cuda/mod.rs:1328-1382): BPTT on the
        device-resident forward state; returns (d_qkv (T,3d), d_gate (T,2H)),
        with the L2-norm and sigmoid backward applied."""
        B, T, H, dh = dev.batch, dev.seq, dev.n_heads, dev.dh
        t_len, d = B * T, H * dh
        if d_o.shape != (t_len, d):
            raise ValueError(f"delta_bwd_dev: d_o has shape {d_o.shape}, expected {(t_len, d)}")
        ddo, dqn, dkn = DevBuf.from_host(d_o), DevBuf.from_host(qnorm), DevBuf.from_host(knorm)
        g_qkv, g_gate = DevBuf(t_len * 3 * d * 4), DevBuf(t_len * 2 * H * 4)
        try:
            _lib.call("asca_delta_bwd_fused", _vp(dev.q), _vp(dev.k), _vp(dev.v), _vp(dev.alpha),
                      _vp(dev.beta), _vp(dqn), _vp(dkn), _vp(ddo), _vp(dev.ws), _vp(g_qkv), _vp(g_gate),
                      B, T, H, dh, None)
            _lib.call("asca_sync")
            d_qkv = g_qkv.to_host((t_len, 3 * d))
            d_gate = g_gate.to_host((t_len, 2 * H))
        finally:
            for b in (ddo, dqn, dkn, g_qkv, g_gate):
                b.free()
        return d_qkv, d_gate

    def delta_bwd_raw(self, dev: DeltaDev, d_o):
        """Raw per-head gradients (dq, dk, dv, dalpha, dbeta) of the recurrence,
        before the L2-norm and sigmoid backward (rust/src/delta.rs:475-587)."""
        B, T, H, dh = dev.batch, dev.seq, dev.n_heads, dev.dh
        t_len, d = B * T, H * dh
        ddo = DevBuf.from_host(d_o)
        outs = [DevBuf(t_len * d * 4) for _ in range(3)] + [DevBuf(t_len * H * 4) for _ in range(2)]
        try:
            _lib.call("asca_delta_bwd_raw", _vp(dev.q), _vp(dev.k), _vp(dev.v), _vp(dev.alpha), _vp(dev.beta),
                      _vp(ddo), _vp(dev.ws), *[_vp(o) for o in outs], B, T, H, dh, None)
            _lib.call("asca_sync")
            res = [o.to_host((t_len, d)) for o in outs[:3]] + [o.to_host((t_len, H)) for o in outs[3:]]
        finally:
            for b in [ddo, *outs]:
                b.free()
        return tuple(res)


    # -- decode -------------------------------------------------------------
    def new_decode_states(self, n_seq: int, n_heads: int, dh: int) -> DevBuf:
        """Zeroed device states (n_seq, H, dh, dh) for delta_decode_step; the
        device counterpart of Model::new_decode_state (rust/src/model.rs:619)."""
        buf = DevBuf(n_seq * n_heads * dh * dh * 4)
        _lib.call("asca_memset32", _vp(buf), 0, C.c_size_t(n_seq * n_heads * dh * dh), None)
        return buf

    def delta_decode_step(self, states: DevBuf, qkv, gate, n_heads: int, dh: int):
        """One token of DeltaBlock::step's state math (rust/src/delta.rs:356-407)
        for every row of qkv (n_seq, 3d) / gate (n_seq, 2H); states stay on the
        device and are updated in place; returns o (n_seq, d) on the host."""
        n = qkv.shape[0]
        d = n_heads * dh
        if qkv.shape != (n, 3 * d) or gate.shape != (n, 2 * n_heads):
            raise ValueError(f"delta_decode_step: qkv {qkv.shape}, gate {gate.shape} for H={n_heads} dh={dh}")
        dq, dg, do = DevBuf.from_host(qkv), DevBuf.from_host(gate), DevBuf(n * d * 4)
        try:
            _lib.call("asca_delta_decode_step", _vp(states), _vp(dq), _vp(dg), _vp(do), n, n_heads, dh, None)
            _lib.call("asca_sync")
            return do.to_host((n, d))
        finally:
            for b in (dq, dg, do):
                b.free()


# --------------------------------------------------------- module functions


def _init_gpu():
    with _gpu_lock:
        if _gpu_state["done"]:
            return _gpu_state["gpu"]
        _gpu_state["done"] = True
        try:
            lib = _lib.load()
        except (ImportError, OSError) as e:
            _gpu_state["err"] = str(e)
            return None
        try:
            _lib.call("asca_init", 0)
            buf = C.create_string_buffer(256)
            _lib.call("asca_describe", buf, 256)
            desc = buf.value.decode()
            cus = int(desc.rsplit(",", 1)[-1].split()[0]) if "CUs" in desc else 0
            _gpu_state["gpu"] = Gpu(desc.split(" (")[0], cus)
            _gpu_state["desc"] = desc
        except AscaError as e:
            _gpu_state["err"] = str(e)
        del lib
        return _gpu_state["gpu"]


def gpu() -> Gpu | None:
    """rust/src/cuda/mod.rs:1494-1496."""
    if _gpu_state["done"]:
        return _gpu_state["gpu"]
    return _init_gpu()


def available() -> bool:
    """rust/src/cuda/mod.rs:1508-1515."""
    return _f().enabled and gpu() is not None


def set_enabled(v: bool) -> None:
    """rust/src/cuda/mod.rs:1517-1519."""
    _f().enabled = bool(v)


def offload(component: str) -> bool:
    """rust/src/cuda/mod.rs:1553-1566 (ASCA_GPU_OFF)."""
    return available() and component.lower() not in _f().off


def offload_opt_in(component: str) -> bool:
    """rust/src/cuda/mod.rs:1537-1551 (ASCA_GPU_ON)."""
    return available() and component.lower() in _f().on


def worth_offload(m: int, k: int, n: int) -> bool:
    """rust/src/cuda/mod.rs:1581-1596 (ASCA_GPU_MIN)."""
    return m * k * n >= _f().min_flops


def describe() -> str:
    """rust/src/cuda/mod.rs:1525-1533."""
    g = gpu()
    if g is not None:
        return f"GPU: {_gpu_state.get('desc', g.name)} ({ARCH}, hipcc)"
    err = _gpu_state.get("err")
    return f"GPU: unavailable (target {ARCH})" + (f" - {err}" if err else "")


def reset_stats() -> None:
    """rust/src/cuda/mod.rs:29-33."""
    _lib.call("asca_reset_stats")


def stats() -> tuple[int, int, int]:
    h2d, d2h, launches = C.c_uint64(), C.c_uint64(), C.c_uint64()
    _lib.call("asca_stats", C.byref(h2d), C.byref(d2h), C.byref(launches))
    return h2d.value, d2h.value, launches.value


def stats_report(steps: int) -> str:
    """rust/src/cuda/mod.rs:76-87."""
    h2d, d2h, l = stats()
    s = max(steps, 1)
    h, dd = h2d / 1e6, d2h / 1e6
    return (f"GPU traffic: H2D {h:.1f} MB, D2H {dd:.1f} MB, {l} kernels "
            f"({h / s:.2f} MB + {dd / s:.2f} MB + {l / s:.0f} kernels per step)")


def fail_after(n: int) -> None:
    """Fault injection: the n-th launch from now fails (-1 disables)."""
    _lib.call("asca_fail_after", C.c_int64(n))
