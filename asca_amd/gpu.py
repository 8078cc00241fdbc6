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
KERNELS = ("delta_fwd", "delta_bwd", "delta_states", "delta_decode", "rmsnorm", "rmsnorm_bwd", "adamw",
           "hash_route", "gather_rows", "scatter_rows", "colsum", "cross_entropy", "gemm", "moe_fwd", "moe_bwd",
           "chunk_fwd", "chunk_bwd", "model_train_step")
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

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DevBuf":
        """Upload keeping the array's dtype (index and id buffers)."""
        a = np.ascontiguousarray(arr)
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


class MoeDev:
    """HashMoE forward state kept on the device for the backward
    (rust/src/cuda/mod.rs:1416-1431): xn, w1, w2, the expert-sorted pre and
    hidden activations and the bucketing (perm, offsets)."""

    def __init__(self, xn, w1, w2, pre, hidden, perm, offsets, t_len, d, d_ff, n_experts):
        self.xn, self.w1, self.w2, self.pre, self.hidden = xn, w1, w2, pre, hidden
        self.perm, self.offsets = perm, offsets
        self.t_len, self.d, self.d_ff, self.n_experts = t_len, d, d_ff, n_experts

    def buckets(self) -> tuple[np.ndarray, np.ndarray]:
        perm = self.perm.to_host((self.t_len,), np.int32)
        off = self.offsets.to_host((self.n_experts + 1,), np.int32)
        return perm, off

    def download_pre_hidden(self) -> tuple[list[np.ndarray], list[np.ndarray]]:
        """Per-expert (n_e x d_ff) pre and hidden (rust/src/cuda/mod.rs:1445-1461)."""
        _, off = self.buckets()
        pre = self.pre.to_host((self.t_len, self.d_ff))
        hid = self.hidden.to_host((self.t_len, self.d_ff))
        return ([pre[off[e]:off[e + 1]] for e in range(self.n_experts)],
                [hid[off[e]:off[e + 1]] for e in range(self.n_experts)])


class MoeBwd:
    """Gradients of the MoE backward (rust/src/cuda/mod.rs:1433-1440)."""

    def __init__(self, d_w1, d_b1, d_w2, d_b2, dxn):
        self.d_w1, self.d_b1, self.d_w2, self.d_b2, self.dxn = d_w1, d_b1, d_w2, d_b2, dxn


class LogitsDev:
    """Head logits kept on the device between the head forward and the
    cross-entropy backward (rust/src/cuda/mod.rs:1398-1408): the (T x vocab)
    logits and the (T x d) h_final that the d_head GEMM reads again."""

    def __init__(self, logits: DevBuf, h_final: DevBuf, t_len: int, vocab: int, d: int):
        self.logits, self.h_final = logits, h_final
        self.t_len, self.vocab, self.d = t_len, vocab, d

    def to_host(self) -> np.ndarray:
        """The logits as a (T x vocab) host matrix (rust/src/cuda/mod.rs:1463-1471)."""
        return self.logits.to_host((self.t_len, self.vocab))

    def free(self) -> None:
        self.logits.free()
        self.h_final.free()


def _mat(x, name, shape=None) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=_f32)
    if shape is not None and a.shape != tuple(shape):
        raise ValueError(f"{name} has shape {a.shape}, expected {tuple(shape)}")
    return a


def _buckets_csr(buckets, t_len: int) -> tuple[np.ndarray, np.ndarray]:
    perm = np.fromiter((t for rows in buckets for t in rows), dtype=np.int32, count=sum(len(r) for r in buckets))
    if perm.size != t_len or (t_len and not np.array_equal(np.sort(perm), np.arange(t_len))):
        raise ValueError("buckets must partition the token rows")
    off = np.zeros(len(buckets) + 1, dtype=np.int32)
    off[1:] = np.cumsum([len(r) for r in buckets])
    return perm, off


_param_dev: dict = {}


def param_key(m: np.ndarray) -> tuple[int, int]:
    """Identity of a parameter's moment buffer (rust/src/cuda/mod.rs:57-62)."""
    return (m.ctypes.data, m.size)


def param_moments(key) -> tuple[np.ndarray, np.ndarray] | None:
    """Device-resident AdamW moments of a parameter, downloaded
    (rust/src/cuda/mod.rs:64-73)."""
    ent = _param_dev.get(key)
    if ent is None:
        return None
    dm, dv, n = ent
    _lib.call("asca_sync")
    return dm.to_host((n,)), dv.to_host((n,))


def reset_param_cache() -> None:
    """rust/src/cuda/mod.rs:50-55."""
    _param_dev.clear()


def to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    b = np.ascontiguousarray(x, dtype=_f32).view(np.uint32)
    return ((b + (0x7FFF + ((b >> 16) & 1))) >> 16).astype(np.uint16)


def from_bf16(x: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 (exact)."""
    return (np.ascontiguousarray(x, dtype=np.uint16).astype(np.uint32) << 16).view(_f32)


class ChunkDev:
    """Chunked-form forward state on the device: the bf16 q, k, v and the
    workspace holding every per-chunk intermediate the backward reads (the
    inputs stay resident for the backward, as DeltaDev keeps them,
    rust/src/cuda/mod.rs:1386-1397)."""

    def __init__(self, ws, inputs, batch, seq, n_heads, dh, chunk):
        self.ws = ws
        self.inputs = inputs
        self.batch, self.seq, self.n_heads, self.dh, self.chunk = batch, seq, n_heads, dh, chunk

    def free(self) -> None:
        for b in (self.ws, *self.inputs):
            b.free()
        self.inputs = ()


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


    # -- row operations -----------------------------------------------------
    def rmsnorm(self, x, eps: float):
        """Gpu::rmsnorm (rust/src/cuda/mod.rs:911-939): (y, inv_rms)."""
        x = _mat(x, "x")
        rows, cols = x.shape
        dx, dy, dinv = DevBuf.from_host(x), DevBuf(x.nbytes), DevBuf(rows * 4)
        try:
            _lib.call("asca_rmsnorm", _vp(dx), _vp(dy), _vp(dinv), rows, cols, eps, None)
            _lib.call("asca_sync")
            return dy.to_host((rows, cols)), dinv.to_host((rows,))
        finally:
            for b in (dx, dy, dinv):
                b.free()

    def rmsnorm_bwd(self, x, dy, eps: float):
        """Gpu::rmsnorm_bwd (rust/src/cuda/mod.rs:1122-1153)."""
        x = _mat(x, "x")
        dy = _mat(dy, "dy", x.shape)
        bx, bdy, bdx = DevBuf.from_host(x), DevBuf.from_host(dy), DevBuf(x.nbytes)
        try:
            _lib.call("asca_rmsnorm_bwd", _vp(bx), _vp(bdy), _vp(bdx), x.shape[0], x.shape[1], eps, None)
            _lib.call("asca_sync")
            return bdx.to_host(x.shape)
        finally:
            for b in (bx, bdy, bdx):
                b.free()

    def cross_entropy_bwd(self, logits, targets):
        """Gpu::cross_entropy_bwd (rust/src/cuda/mod.rs:945-997): (mean loss,
        dlogits); the loss is the f32 sum of per-row losses times 1/T."""
        logits = _mat(logits, "logits")
        t_len, v = logits.shape
        tg = np.ascontiguousarray(targets, dtype=np.uint32)
        if tg.shape != (t_len,):
            raise ValueError("targets len must equal logits rows")
        bl, bt, bd, bs = DevBuf.from_host(logits), DevBuf.from_array(tg), DevBuf(logits.nbytes), DevBuf(t_len * 4)
        try:
            _lib.call("asca_cross_entropy", _vp(bl), _vp(bt), t_len, v, _vp(bd), _vp(bs), None)
            _lib.call("asca_sync")
            losses = bs.to_host((t_len,))
            inv_t = _f32(1.0) / _f32(t_len)
            loss = (np.cumsum(losses, dtype=_f32)[-1] if t_len else _f32(0)) * inv_t
            return float(loss), bd.to_host((t_len, v))
        finally:
            for b in (bl, bt, bd, bs):
                b.free()

    # -- output head, logits resident ----------------------------------------
    def head_forward_dev(self, h_final, head) -> LogitsDev:
        """Gpu::head_forward_dev (rust/src/cuda/mod.rs:826-845): logits =
        h_final @ head on the matrix cores, left on the device."""
        h = _mat(h_final, "h_final")
        t_len, d = h.shape
        w = _mat(head, "head")
        if w.shape[0] != d:
            raise ValueError(f"head_forward_dev: head has {w.shape[0]} rows, h_final {d} columns")
        v = w.shape[1]
        dh, dw, dl = DevBuf.from_host(h), DevBuf.from_host(w), DevBuf(t_len * v * 4)
        try:
            _lib.call("asca_gemm", 0, 0, t_len, v, d, 1.0, _vp(dh), d, _vp(dw), v, 0.0, _vp(dl), v, None, None)
            _lib.call("asca_sync")
        except BaseException:
            dh.free()
            dl.free()
            raise
        finally:
            dw.free()
        return LogitsDev(dl, dh, t_len, v, d)

    def head_bwd_dev(self, dev: LogitsDev, targets, head_t):
        """Gpu::head_bwd_dev (rust/src/cuda/mod.rs:847-908): cross-entropy
        backward on the resident logits, then d_head = h_final^T @ dlogits and
        dh = dlogits @ head_t, dlogits never leaving the device.  Returns
        (mean loss, d_head (d x vocab), dh (T x d)); the loss is the f32 sum
        of the per-row losses times 1/T."""
        t_len, v, d = dev.t_len, dev.vocab, dev.d
        tg = np.ascontiguousarray(targets, dtype=np.uint32)
        if tg.shape != (t_len,):
            raise ValueError("head_bwd_dev: targets len must equal the logits rows")
        ht = _mat(head_t, "head_t")
        if ht.shape[0] != v:
            raise ValueError("head_bwd_dev: head_t must be (vocab, d)")
        if ht.shape[1] != d:
            raise ValueError(f"head_bwd_dev: head_t has {ht.shape[1]} columns, h_final {d}")
        bt, bht = DevBuf.from_array(tg), DevBuf.from_host(ht)
        bdl, bls, bdw, bdh = DevBuf(t_len * v * 4), DevBuf(t_len * 4), DevBuf(d * v * 4), DevBuf(t_len * d * 4)
        try:
            _lib.call("asca_cross_entropy", _vp(dev.logits), _vp(bt), t_len, v, _vp(bdl), _vp(bls), None)
            _lib.call("asca_gemm", 1, 0, d, v, t_len, 1.0, _vp(dev.h_final), d, _vp(bdl), v, 0.0, _vp(bdw), v,
                      None, None)
            _lib.call("asca_gemm", 0, 0, t_len, d, v, 1.0, _vp(bdl), v, _vp(bht), d, 0.0, _vp(bdh), d, None, None)
            _lib.call("asca_sync")
            losses = bls.to_host((t_len,))
            inv_t = _f32(1.0) / _f32(t_len)
            loss = (np.cumsum(losses, dtype=_f32)[-1] if t_len else _f32(0)) * inv_t
            return float(loss), bdw.to_host((d, v)), bdh.to_host((t_len, d))
        finally:
            for b in (bt, bht, bdl, bls, bdw, bdh):
                b.free()

    def gather_rows(self, src, idx):
        """Gpu::gather_rows (rust/src/cuda/mod.rs:1156-1188): src[idx]."""
        src = _mat(src, "src")
        ix = np.ascontiguousarray(idx, dtype=np.int32)
        if ix.size and (ix.min() < 0 or ix.max() >= src.shape[0]):
            raise ValueError("gather_rows: index out of range")
        bs, bi, bd = DevBuf.from_host(src), DevBuf.from_array(ix), DevBuf(ix.size * src.shape[1] * 4)
        try:
            _lib.call("asca_gather_rows", _vp(bs), _vp(bi), ix.size, src.shape[1], _vp(bd), None)
            _lib.call("asca_sync")
            return bd.to_host((ix.size, src.shape[1]))
        finally:
            for b in (bs, bi, bd):
                b.free()

    def scatter_rows(self, src, idx, dst: np.ndarray) -> None:
        """Gpu::scatter_rows (rust/src/cuda/mod.rs:1190-1222): dst[idx] = src,
        in place on the host matrix."""
        src = _mat(src, "src")
        ix = np.ascontiguousarray(idx, dtype=np.int32)
        if dst.dtype != _f32 or not dst.flags["C_CONTIGUOUS"] or dst.shape[1] != src.shape[1]:
            raise ValueError("scatter_rows: dst must be a C-contiguous float32 matrix with src's columns")
        if ix.size != src.shape[0] or (ix.size and (ix.min() < 0 or ix.max() >= dst.shape[0])):
            raise ValueError("scatter_rows: bad indices")
        if np.unique(ix).size != ix.size:
            raise ValueError("scatter_rows: indices must be distinct")
        bs, bi, bd = DevBuf.from_host(src), DevBuf.from_array(ix), DevBuf.from_host(dst)
        try:
            _lib.call("asca_scatter_rows", _vp(bs), _vp(bi), ix.size, src.shape[1], _vp(bd), None)
            _lib.call("asca_sync")
            bd.download(dst)
        finally:
            for b in (bs, bi, bd):
                b.free()

    # -- GEMM ---------------------------------------------------------------
    def gemm(self, a, b, trans_a: bool = False, trans_b: bool = False, alpha: float = 1.0,
             beta: float = 0.0, c=None, bias=None):
        """C = alpha op(A) op(B) + bias + beta C on the matrix cores."""
        a, b = _mat(a, "a"), _mat(b, "b")
        m, k = (a.shape[1], a.shape[0]) if trans_a else a.shape
        k2, n = (b.shape[1], b.shape[0]) if trans_b else b.shape
        if k != k2:
            raise ValueError(f"gemm: inner dimensions {k} and {k2} differ")
        cc = _mat(c, "c", (m, n)) if c is not None else np.zeros((m, n), dtype=_f32)
        bb = _mat(bias, "bias", (n,)) if bias is not None else None
        ba, bbuf, bc = DevBuf.from_host(a), DevBuf.from_host(b), DevBuf.from_host(cc)
        bbias = DevBuf.from_host(bb) if bb is not None else None
        try:
            _lib.call("asca_gemm", int(trans_a), int(trans_b), m, n, k, alpha, _vp(ba), a.shape[1], _vp(bbuf),
                      b.shape[1], beta, _vp(bc), n, _vp(bbias), None)
            _lib.call("asca_sync")
            return bc.to_host((m, n))
        finally:
            for x in (ba, bbuf, bc, bbias):
                if x is not None:
                    x.free()

    def matmul(self, a, b):
        """Gpu::matmul (rust/src/cuda/mod.rs:286-313): A @ B."""
        return self.gemm(a, b)

    def matmul_ta(self, a, b):
        """Gpu::matmul_ta (rust/src/cuda/mod.rs:316-344): A^T @ B."""
        return self.gemm(a, b, trans_a=True)

    def matmul_t(self, a, b):
        """A @ B^T (Mat::matmul_t, rust/src/tensor.rs:180-201)."""
        return self.gemm(a, b, trans_b=True)

    # -- AdamW ----------------------------------------------------------------
    def adamw_scalars(self, lr, beta1, beta2, eps, wd, step: int):
        """(lr_bc, eps_t, wd_eff) of AdamW::update (rust/src/tensor.rs:392-402), f32."""
        out = (C.c_float * 3)()
        _lib.call("asca_adamw_scalars", lr, beta1, beta2, eps, wd, step, out)
        return out[0], out[1], out[2]

    def adamw_update(self, val: np.ndarray, grad, m: np.ndarray, v: np.ndarray, lr, beta1, beta2, eps_t, wd):
        """Gpu::adamw_update (rust/src/cuda/mod.rs:1057-1119): one update of
        val, m, v in place (host arrays) with the CPU path's element math."""
        n = val.size
        for name, x in (("val", val), ("m", m), ("v", v)):
            if x.dtype != _f32 or not x.flags["C_CONTIGUOUS"] or x.size != n:
                raise ValueError(f"adamw_update: {name} must be a C-contiguous float32 array of {n}")
        g = _mat(grad, "grad").reshape(-1)
        if g.size != n:
            raise ValueError("adamw_update: grad size differs")
        bp, bg, bm, bv = DevBuf.from_host(val), DevBuf.from_host(g), DevBuf.from_host(m), DevBuf.from_host(v)
        try:
            _lib.call("asca_adamw", _vp(bp), _vp(bg), _vp(bm), _vp(bv), n, lr, beta1, beta2, eps_t, wd, None)
            _lib.call("asca_sync")
            bp.download(val)
            bm.download(m)
            bv.download(v)
        finally:
            for b in (bp, bg, bm, bv):
                b.free()

    def adamw_resident(self, key, val: np.ndarray, grad, m0, v0, lr, beta1, beta2, eps_t, wd):
        """Gpu::adamw_resident (rust/src/cuda/mod.rs:1003-1054): moments stay
        on the device between steps (param_moments downloads them)."""
        n = val.size
        ent = _param_dev.get(key)
        if ent is None:
            ent = (DevBuf.from_host(np.asarray(m0).reshape(-1)), DevBuf.from_host(np.asarray(v0).reshape(-1)), n)
            _param_dev[key] = ent
        dm, dv, _ = ent
        g = _mat(grad, "grad").reshape(-1)
        bp, bg = DevBuf.from_host(val), DevBuf.from_host(g)
        try:
            _lib.call("asca_adamw", _vp(bp), _vp(bg), _vp(dm), _vp(dv), n, lr, beta1, beta2, eps_t, wd, None)
            _lib.call("asca_sync")
            bp.download(val)
        finally:
            bp.free()
            bg.free()

    # -- hash MoE ---------------------------------------------------------------
    def hash_route(self, ids, n_experts: int):
        """Expert of every token and the stable buckets as (expert, perm,
        offsets) (rust/src/model.rs:69-77,190-193), computed on the device."""
        ix = np.ascontiguousarray(ids, dtype=np.uint32)
        n = ix.size
        wsb = C.c_size_t()
        _lib.call("asca_hash_route_ws_bytes", n, n_experts, C.byref(wsb))
        bi, be, bp = DevBuf.from_array(ix), DevBuf(n * 4), DevBuf(n * 4)
        bo, bw = DevBuf((n_experts + 1) * 4), DevBuf(wsb.value)
        try:
            _lib.call("asca_hash_route", _vp(bi), n, n_experts, _vp(be), _vp(bp), _vp(bo), _vp(bw), None)
            _lib.call("asca_sync")
            return (be.to_host((n,), np.int32), bp.to_host((n,), np.int32),
                    bo.to_host((n_experts + 1,), np.int32))
        finally:
            for b in (bi, be, bp, bo, bw):
                b.free()

    def moe_forward_dev(self, xn, w1, b1, w2, b2, buckets, d_ff: int):
        """Gpu::moe_forward_dev (rust/src/cuda/mod.rs:523-607): (out, MoeDev)
        with every expert product in one grouped launch each."""
        xn = _mat(xn, "xn")
        t_len, d = xn.shape
        n_experts = len(buckets)
        w1 = _mat(w1, "w1", (d, n_experts * d_ff))
        w2 = _mat(w2, "w2", (n_experts * d_ff, d))
        b1 = _mat(b1, "b1").reshape(-1)
        b2 = _mat(b2, "b2").reshape(-1)
        if b1.size != n_experts * d_ff or b2.size != d:
            raise ValueError("moe_forward_dev: bias sizes")
        perm, off = _buckets_csr(buckets, t_len)
        bx, bw1, bw2 = DevBuf.from_host(xn), DevBuf.from_host(w1), DevBuf.from_host(w2)
        bb1, bb2 = DevBuf.from_host(b1), DevBuf.from_host(b2)
        bperm, boff = DevBuf.from_array(perm), DevBuf.from_array(off)
        pre, hid, out = DevBuf(t_len * d_ff * 4), DevBuf(t_len * d_ff * 4), DevBuf(t_len * d * 4)
        try:
            _lib.call("asca_moe_fwd", _vp(bx), _vp(bw1), _vp(bb1), _vp(bw2), _vp(bb2), _vp(bperm), _vp(boff),
                      t_len, d, d_ff, n_experts, _vp(out), _vp(pre), _vp(hid), None)
            _lib.call("asca_sync")
            o = out.to_host((t_len, d))
        finally:
            for b in (bb1, bb2, out):
                b.free()
        return o, MoeDev(bx, bw1, bw2, pre, hid, bperm, boff, t_len, d, d_ff, n_experts)

    def moe_bwd_dev(self, dev: MoeDev, dout) -> MoeBwd:
        """Gpu::moe_bwd_dev (rust/src/cuda/mod.rs:745-824): all expert
        gradients on the device; the caller applies rmsnorm_bwd to dxn."""
        t_len, d, d_ff, E = dev.t_len, dev.d, dev.d_ff, dev.n_experts
        dout = _mat(dout, "dout", (t_len, d))
        bdo = DevBuf.from_host(dout)
        bdx, bdw1, bdb1 = DevBuf(t_len * d * 4), DevBuf(d * E * d_ff * 4), DevBuf(E * d_ff * 4)
        bdw2, bdb2, bws = DevBuf(E * d_ff * d * 4), DevBuf(d * 4), DevBuf(t_len * d_ff * 4)
        try:
            _lib.call("asca_moe_bwd", _vp(dev.xn), _vp(dev.w1), _vp(dev.w2), _vp(dev.pre), _vp(dev.hidden),
                      _vp(dev.perm), _vp(dev.offsets), _vp(bdo), t_len, d, d_ff, E, _vp(bdx), _vp(bdw1),
                      _vp(bdb1), _vp(bdw2), _vp(bdb2), _vp(bws), 0, None)
            _lib.call("asca_sync")
            return MoeBwd(bdw1.to_host((d, E * d_ff)), bdb1.to_host((E * d_ff,)), bdw2.to_host((E * d_ff, d)),
                          bdb2.to_host((d,)), bdx.to_host((t_len, d)))
        finally:
            for b in (bdo, bdx, bdw1, bdb1, bdw2, bdb2, bws):
                b.free()

    # -- chunked form ---------------------------------------------------------
    def delta_chunked(self, q, k, v, alpha, beta, batch: int, seq: int, n_heads: int, dh: int, chunk: int = 64):
        """Forward of the chunked (WY/UT) form (docs/SPEC_V2.md:50-69) on bf16
        q, k, v (uint16 bit patterns, or float32 rounded to bf16 here) and f32
        gates; returns (o f32, ChunkDev)."""
        d, t_len = n_heads * dh, batch * seq
        bf = [x if x.dtype == np.uint16 else to_bf16(x) for x in (q, k, v)]
        for name, m in zip("qkv", bf):
            if m.shape != (t_len, d):
                raise ValueError(f"delta_chunked: {name} has shape {m.shape}, expected {(t_len, d)}")
        wsb = C.c_size_t()
        _lib.call("asca_chunk_ws_bytes", batch, seq, n_heads, dh, chunk, C.byref(wsb))
        ins = [DevBuf.from_array(x) for x in bf]
        ga, gb = DevBuf.from_host(alpha), DevBuf.from_host(beta)
        ws, out = DevBuf(wsb.value), DevBuf(t_len * d * 4)
        try:
            _lib.call("asca_chunk_fwd", *[_vp(x) for x in ins], _vp(ga), _vp(gb), _vp(out), _vp(ws), batch, seq,
                      n_heads, dh, chunk, None)
            _lib.call("asca_sync")
            o = out.to_host((t_len, d))
        except Exception:
            for x in (*ins, ws):
                x.free()
            raise
        finally:
            for x in (ga, gb, out):
                x.free()
        return o, ChunkDev(ws, tuple(ins), batch, seq, n_heads, dh, chunk)

    def delta_chunked_bwd(self, dev: ChunkDev, d_o):
        """Raw gradients (dq, dk, dv, dalpha, dbeta) of the chunked form given
        dO (bf16 bit patterns or float32 rounded to bf16)."""
        B, T, H, dh, Cc = dev.batch, dev.seq, dev.n_heads, dev.dh, dev.chunk
        t_len, d = B * T, H * dh
        x = d_o if d_o.dtype == np.uint16 else to_bf16(d_o)
        bdo = DevBuf.from_array(x)
        outs = [DevBuf(t_len * d * 4) for _ in range(3)] + [DevBuf(t_len * H * 4) for _ in range(2)]
        try:
            _lib.call("asca_chunk_bwd", *[_vp(x) for x in dev.inputs], _vp(bdo), _vp(dev.ws),
                      *[_vp(o) for o in outs], B, T, H, dh, Cc, None)
            _lib.call("asca_sync")
            return tuple([o.to_host((t_len, d)) for o in outs[:3]] + [o.to_host((t_len, H)) for o in outs[3:]])
        finally:
            for b in (bdo, *outs):
                b.free()

    def delta_chunked_f32(self, q, k, v, alpha, beta, batch: int, seq: int, n_heads: int, dh: int,
                          chunk: int = 32):
        """Forward of the chunked form on f32 q, k, v (asca_chunk_fwd_f32, the
        batched-GEMM path at any chunk size); returns (o f32, ChunkDev).  The
        workspace keeps f32 copies of q, k, v, so the backward takes only dO."""
        d, t_len = n_heads * dh, batch * seq
        for name, m in zip("qkv", (q, k, v)):
            if m.shape != (t_len, d):
                raise ValueError(f"delta_chunked_f32: {name} has shape {m.shape}, expected {(t_len, d)}")
        wsb = C.c_size_t()
        _lib.call("asca_chunk_ws_bytes_f32", batch, seq, n_heads, dh, chunk, C.byref(wsb))
        ins = [DevBuf.from_host(x) for x in (q, k, v, alpha, beta)]
        ws, out = DevBuf(wsb.value), DevBuf(t_len * d * 4)
        try:
            _lib.call("asca_chunk_fwd_f32", *[_vp(x) for x in ins], _vp(out), _vp(ws), batch, seq, n_heads, dh,
                      chunk, None)
            _lib.call("asca_sync")
            o = out.to_host((t_len, d))
        except Exception:
            ws.free()
            raise
        finally:
            for x in (*ins, out):
                x.free()
        return o, ChunkDev(ws, (), batch, seq, n_heads, dh, chunk)

    def delta_chunked_f32_bwd(self, dev: ChunkDev, d_o):
        """Raw gradients (dq, dk, dv, dalpha, dbeta) of delta_chunked_f32 given
        f32 dO."""
        B, T, H, dh, Cc = dev.batch, dev.seq, dev.n_heads, dev.dh, dev.chunk
        t_len, d = B * T, H * dh
        bdo = DevBuf.from_host(d_o)
        outs = [DevBuf(t_len * d * 4) for _ in range(3)] + [DevBuf(t_len * H * 4) for _ in range(2)]
        try:
            _lib.call("asca_chunk_bwd_f32", _vp(bdo), _vp(dev.ws), *[_vp(o) for o in outs], B, T, H, dh, Cc, None)
            _lib.call("asca_sync")
            return tuple([o.to_host((t_len, d)) for o in outs[:3]] + [o.to_host((t_len, H)) for o in outs[3:]])
        finally:
            for b in (bdo, *outs):
                b.free()

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
