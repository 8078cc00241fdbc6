"""Device-resident ASCA model over libasca_hip (asca_model_* in the C ABI).

The host-side shape of the reference's Model (rust/src/model.rs:528-802) and
training step (rust/src/train.rs:176-186): `forward_backward` is zero_grads +
forward + backward, `adamw` is the optimiser step over every tensor, and
`train_step` both; `new_decode_state` / `step` are Model::new_decode_state /
Model::step (model.rs:619-649) for many sequences at once.  Parameters, gradients and AdamW moments stay on the device;
`params()` / `grads()` / `set_params()` move them as host arrays in the
reference's params() order for initialisation, checkpoints and parity checks.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .gpu import DevBuf, _vp, describe, gpu

_f32 = np.float32


class DeviceModel:
    def __init__(self, vocab: int, d_model: int, n_heads: int, n_layers: int, n_experts: int, d_ff: int):
        if gpu() is None:  # lazy device initialisation, as crate::cuda::gpu() does
            raise RuntimeError(describe())
        h = C.c_void_p()
        _lib.call("asca_model_create", vocab, d_model, n_heads, n_layers, n_experts, d_ff, C.byref(h))
        self._h = h
        self.vocab, self.d_model, self.n_heads = vocab, d_model, n_heads
        self.n_layers, self.n_experts, self.d_ff = n_layers, n_experts, d_ff
        n = C.c_int()
        _lib.call("asca_model_num_tensors", h, C.byref(n))
        self.tensors = []
        name = C.create_string_buffer(64)
        for i in range(n.value):
            off, r, c = C.c_size_t(), C.c_int(), C.c_int()
            _lib.call("asca_model_tensor_info", h, i, name, 64, C.byref(off), C.byref(r), C.byref(c))
            self.tensors.append((name.value.decode(), off.value, r.value, c.value))
        nf = C.c_size_t()
        ptrs = [C.c_void_p() for _ in range(4)]
        _lib.call("asca_model_buffers", h, C.byref(nf), *[C.byref(p) for p in ptrs])
        self.n_floats = nf.value
        self._ptr = {k: p.value for k, p in zip(("params", "grads", "m", "v"), ptrs)}
        self._bufs: dict = {}

    def num_params(self) -> int:
        return sum(r * c for _, _, r, c in self.tensors)

    # -- host <-> device copies in params() order --------------------------------
    def _get(self, which: str) -> list[np.ndarray]:
        _lib.call("asca_sync")
        flat = np.empty(self.n_floats, dtype=_f32)
        _lib.call("asca_d2h", flat.ctypes.data_as(C.c_void_p), C.c_void_p(self._ptr[which]),
                  C.c_size_t(flat.nbytes))
        return [flat[off:off + r * c].reshape(r, c).copy() for _, off, r, c in self.tensors]

    def _set(self, which: str, arrays) -> None:
        arrays = list(arrays)
        if len(arrays) != len(self.tensors):
            raise ValueError(f"expected {len(self.tensors)} tensors, got {len(arrays)}")
        flat = np.zeros(self.n_floats, dtype=_f32)
        for (name, off, r, c), a in zip(self.tensors, arrays):
            a = np.asarray(a, dtype=_f32)
            if a.size != r * c:
                raise ValueError(f"{name}: {a.size} values for a {r}x{c} tensor")
            flat[off:off + r * c] = a.reshape(-1)
        _lib.call("asca_sync")
        _lib.call("asca_h2d", C.c_void_p(self._ptr[which]), flat.ctypes.data_as(C.c_void_p), C.c_size_t(flat.nbytes))

    def params(self):
        return self._get("params")

    def grads(self):
        return self._get("grads")

    def moments(self):
        return self._get("m"), self._get("v")

    def set_params(self, arrays) -> None:
        self._set("params", arrays)

    def set_grads(self, arrays) -> None:
        self._set("grads", arrays)

    def set_moments(self, m, v) -> None:
        self._set("m", m)
        self._set("v", v)

    # -- optimiser ---------------------------------------------------------------
    def set_adamw(self, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.01, step: int = 0) -> None:
        """AdamW::new defaults (rust/src/tensor.rs:381-390); `step` is the shared
        counter that advances once per tensor per optimiser step."""
        _lib.call("asca_model_set_adamw", self._h, lr, beta1, beta2, eps, wd, step)

    def adamw_step_count(self) -> int:
        s = C.c_uint32()
        _lib.call("asca_model_adamw_step_count", self._h, C.byref(s))
        return s.value

    # -- steps -----------------------------------------------------------------
    def _ids(self, key: str, a) -> DevBuf:
        a = np.ascontiguousarray(a, dtype=np.uint32)
        buf = self._bufs.get(key)
        if buf is None or buf.nbytes < a.nbytes:
            buf = DevBuf(a.nbytes)
            self._bufs[key] = buf
        buf.upload(a)
        return buf

    def upload_batch(self, ids, targets):
        """Device copies of ids / targets (reused across calls)."""
        return self._ids("ids", ids), self._ids("tgt", targets)

    def _loss_buf(self) -> DevBuf:
        if "loss" not in self._bufs:
            self._bufs["loss"] = DevBuf(4)
        return self._bufs["loss"]

    def forward_backward(self, ids, targets, batch: int, sync: bool = True):
        n = len(ids)
        if n % batch or len(targets) != n:
            raise ValueError("ids/targets must hold batch * seq tokens each")
        di, dt = self.upload_batch(ids, targets)
        return self.forward_backward_dev(di, dt, batch, n // batch, sync)

    def forward_backward_dev(self, ids: DevBuf, targets: DevBuf, batch: int, seq: int, sync: bool = True,
                             stream=None):
        lb = self._loss_buf()
        _lib.call("asca_model_forward_backward", self._h, _vp(ids), _vp(targets), batch, seq, _vp(lb), stream)
        return self._read_loss() if sync else None

    def adamw(self, stream=None) -> None:
        _lib.call("asca_model_adamw", self._h, stream)

    def train_step(self, ids, targets, batch: int, sync: bool = True):
        di, dt = self.upload_batch(ids, targets)
        return self.train_step_dev(di, dt, batch, len(ids) // batch, sync)

    def train_step_dev(self, ids: DevBuf, targets: DevBuf, batch: int, seq: int, sync: bool = True, stream=None):
        lb = self._loss_buf()
        _lib.call("asca_model_train_step", self._h, _vp(ids), _vp(targets), batch, seq, _vp(lb), stream)
        return self._read_loss() if sync else None

    # -- decode (Model::new_decode_state / Model::step, model.rs:619-649) -----
    def decode_state_floats(self) -> int:
        """Floats of carried state per sequence: n_layers * n_heads * dh * dh."""
        n = C.c_size_t()
        _lib.call("asca_model_decode_state_floats", self._h, C.byref(n))
        return n.value

    def new_decode_state(self, n_seq: int = 1) -> DevBuf:
        """Zero states for n_seq new sequences, layout (L, n_seq, H, dh, dh)."""
        buf = DevBuf(4 * n_seq * self.decode_state_floats())
        _lib.call("asca_memset32", _vp(buf), 0, n_seq * self.decode_state_floats(), None)
        return buf

    def step(self, ids, states: DevBuf, sync: bool = True):
        """One token per sequence (ids: n_seq ints) through the model on the
        carried states; returns the (n_seq, V) logits (None with sync=False:
        they stay in the device buffer `decode_logits`)."""
        ids = np.ascontiguousarray(np.atleast_1d(ids), dtype=np.uint32)
        n = len(ids)
        if states.nbytes < 4 * n * self.decode_state_floats():
            raise ValueError("states buffer too small for %d sequences" % n)
        di = self._ids("dec_ids", ids)
        lb = self._bufs.get("decode_logits")
        if lb is None or lb.nbytes < 4 * n * self.vocab:
            lb = DevBuf(4 * n * self.vocab)
            self._bufs["decode_logits"] = lb
        _lib.call("asca_model_decode_step", self._h, _vp(di), n, _vp(states), _vp(lb), None)
        if not sync:
            return None
        _lib.call("asca_sync")
        return lb.to_host((n, self.vocab))

    def _read_loss(self) -> float:
        _lib.call("asca_sync")
        return float(self._loss_buf().to_host((1,))[0])

    def close(self) -> None:
        if self._h:
            for b in self._bufs.values():
                b.free()
            self._bufs.clear()
            _lib.call("asca_model_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
