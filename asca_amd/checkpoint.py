"""Checkpoints of the device-resident model in the reference's file formats.

rust/src/train.rs:290-540 defines two little-endian formats, both with the
tensors in params() order (embed, head, then per layer w_qkv, b_qkv, w_gate,
b_gate, w_o, b_o, w1, b1, w2, b2):

  ASCA2CK1 (save / load, weights only):
      magic, 6 x u64 config (vocab, d_model, n_heads, n_layers, n_experts,
      d_ff), then per tensor u64 numel + numel f32 values.
  ASCARSM1 (save_resume / load_resume, resumable):
      magic, 6 x u64 config, u64 training step, then per tensor u64 numel +
      numel f32 values + numel f32 AdamW m + numel f32 AdamW v.

The reference writes the moments the optimiser actually uses, fetching them
from VRAM when they live there (train.rs:320-331, cuda::param_moments); here
they always live in HBM and are read from the model's moment buffers.  A
resume sets the AdamW counter to the saved training step, as load_resume does
(train.rs:451-452), and an ASCA2CK1 file resumes at step 0 (train.rs:399-403).
save_resume writes atomically: <path>.tmp, fsync, rename (train.rs:297-346).
"""
from __future__ import annotations

import os
import struct

import numpy as np

MAGIC = b"ASCA2CK1"
MAGIC_R = b"ASCARSM1"
_f32 = np.dtype("<f4")


class CheckpointError(ValueError):
    """A file that is not a checkpoint of these formats, or is truncated
    (the reference's io::ErrorKind::InvalidData)."""


def _need(buf: bytes, off: int, n: int) -> None:
    # train.rs:347-359: a truncated file is a readable error, not a crash
    if off + n > len(buf):
        raise CheckpointError(f"truncated checkpoint: need {n} bytes at offset {off}, file size {len(buf)}")


# -- pure format (host arrays) ---------------------------------------------------
def encode_resume(cfg, step: int, params, m, v) -> bytes:
    """ASCARSM1 bytes (train.rs:303-339)."""
    out = [MAGIC_R, struct.pack("<6Q", *cfg), struct.pack("<Q", step)]
    for p, mm, vv in zip(params, m, v):
        n = p.size
        out.append(struct.pack("<Q", n))
        for a in (p, mm, vv):
            a = np.ascontiguousarray(a, dtype=_f32).reshape(-1)
            if a.size != n:
                raise ValueError("moment size differs from its tensor")
            out.append(a.tobytes())
    return b"".join(out)


def encode_weights(cfg, params) -> bytes:
    """ASCA2CK1 bytes (train.rs:457-478)."""
    out = [MAGIC, struct.pack("<6Q", *cfg)]
    for p in params:
        out.append(struct.pack("<Q", p.size))
        out.append(np.ascontiguousarray(p, dtype=_f32).reshape(-1).tobytes())
    return b"".join(out)


def peek(buf: bytes):
    """(cfg, step) of an ASCARSM1 header (peek_resume, train.rs:361-387)."""
    if len(buf) < 64 or buf[:8] != MAGIC_R:
        raise CheckpointError("not a resumable checkpoint (no ASCARSM1 header); the step is unknown")
    return tuple(struct.unpack_from("<6Q", buf, 8)), struct.unpack_from("<Q", buf, 56)[0]


def decode(buf: bytes, shapes):
    """(cfg, step, params, m, v) from either format; `shapes(cfg)` gives the
    tensor shapes of that config in params() order.  A weights-only file has
    step 0 and zero moments (load_resume, train.rs:389-455; load, :480-540)."""
    if len(buf) < 8:
        raise CheckpointError("checkpoint too small")
    magic = buf[:8]
    if magic not in (MAGIC, MAGIC_R):
        raise CheckpointError("not an ASCA v2 checkpoint")
    resume = magic == MAGIC_R
    off = 8
    _need(buf, off, 48)
    cfg = tuple(struct.unpack_from("<6Q", buf, off))
    off += 48
    step = 0
    if resume:
        _need(buf, off, 8)
        step = struct.unpack_from("<Q", buf, off)[0]
        off += 8
    params, m, v = [], [], []
    for i, shape in enumerate(shapes(cfg)):
        _need(buf, off, 8)
        n = struct.unpack_from("<Q", buf, off)[0]
        off += 8
        want = int(np.prod(shape))
        parts = []
        for _ in range(3 if resume else 1):
            _need(buf, off, 4 * n)
            parts.append(np.frombuffer(buf, dtype=_f32, count=n, offset=off).astype(np.float32))
            off += 4 * n
        if n != want:
            raise CheckpointError(f"param {i} size mismatch: {n} vs {want}")
        params.append(parts[0].reshape(shape))
        m.append(parts[1].reshape(shape) if resume else np.zeros(shape, np.float32))
        v.append(parts[2].reshape(shape) if resume else np.zeros(shape, np.float32))
    return cfg, step, params, m, v


def write_atomic(path: str, data: bytes) -> None:
    """<path>.tmp, flush + fsync, then rename: a reader sees the old file or the
    new one, never a mix (train.rs:297-302,340-345)."""
    tmp = f"{path}.tmp"
    with open(tmp, "wb") as f:
        f.write(data)
        f.flush()
        os.fsync(f.fileno())
    os.replace(tmp, path)


def model_shapes(cfg):
    """Tensor shapes of a config, params() order (model.rs:596-603)."""
    V, d, H, L, E, dff = (int(x) for x in cfg)
    s = [(V, d), (d, V)]
    for _ in range(L):
        s += [(d, 3 * d), (1, 3 * d), (d, 2 * H), (1, 2 * H), (d, d), (1, d), (d, E * dff), (1, E * dff),
              (E * dff, d), (1, d)]
    return s


# -- the device-resident model ---------------------------------------------------
def _cfg(model):
    return (model.vocab, model.d_model, model.n_heads, model.n_layers, model.n_experts, model.d_ff)


def save_resume(path: str, model, step: int) -> None:
    """train::save_resume for a DeviceModel: weights and the AdamW moments
    read back from HBM, plus the training step."""
    m, v = model.moments()
    write_atomic(path, encode_resume(_cfg(model), step, model.params(), m, v))


def save(path: str, model) -> None:
    """train::save (weights only)."""
    with open(path, "wb") as f:
        f.write(encode_weights(_cfg(model), model.params()))


def peek_resume(path: str):
    """train::peek_resume: (config, step) from the header only."""
    with open(path, "rb") as f:
        return peek(f.read(64))


def load_resume(path: str):
    """train::load_resume: a new DeviceModel holding the file's weights and
    moments, AdamW counter = the saved step; returns (model, step)."""
    from .model import DeviceModel

    with open(path, "rb") as f:
        buf = f.read()
    cfg, step, params, m, v = decode(buf, model_shapes)
    model = DeviceModel(*(int(x) for x in cfg))
    model.set_params(params)
    model.set_moments(m, v)
    model.set_adamw(step=step)
    return model, step


def load(path: str):
    """train::load: a DeviceModel from either format (weights only)."""
    model, _ = load_resume(path)
    return model
