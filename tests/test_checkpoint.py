"""Checkpoint formats of the reference (rust/src/train.rs:290-540) on host
arrays: ASCARSM1 (weights + AdamW moments + step) and ASCA2CK1 (weights).

The reference ships no checkpoint file, so the layout is pinned by what its
reader fixes: peek_resume reads the step at bytes 56..64 (train.rs:375), the
tensors follow in params() order with a u64 count each, and a truncated file
is an error at every cut (train.rs:347-359)."""
import os
import struct

import numpy as np
import pytest

from asca_amd import checkpoint as ck

CFG = (256, 16, 2, 2, 3, 8)   # vocab, d_model, n_heads, n_layers, n_experts, d_ff


def _tensors(seed, cfg=CFG):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal(s).astype(np.float32) for s in ck.model_shapes(cfg)]


def test_model_shapes_follow_params_order():
    s = ck.model_shapes(CFG)
    assert len(s) == 2 + 10 * CFG[3]
    assert s[0] == (256, 16) and s[1] == (16, 256)
    assert s[2:12] == [(16, 48), (1, 48), (16, 4), (1, 4), (16, 16), (1, 16), (16, 24), (1, 24), (24, 16), (1, 16)]


def test_resume_round_trip_and_layout():
    p, m, v = _tensors(1), _tensors(2), _tensors(3)
    buf = ck.encode_resume(CFG, 1234, p, m, v)
    # 8 magic + 48 config + 8 step, then per tensor a count and three arrays
    assert len(buf) == 64 + sum(8 + 12 * a.size for a in p)
    assert buf[:8] == b"ASCARSM1"
    assert struct.unpack_from("<Q", buf, 56)[0] == 1234
    assert struct.unpack_from("<Q", buf, 64)[0] == p[0].size
    assert ck.peek(buf) == (CFG, 1234)
    cfg, step, p2, m2, v2 = ck.decode(buf, ck.model_shapes)
    assert cfg == CFG and step == 1234
    for a, b in zip(p + m + v, p2 + m2 + v2):
        np.testing.assert_array_equal(a, b)
    # the first tensor's values start right after its count, its m after them
    np.testing.assert_array_equal(np.frombuffer(buf, "<f4", p[0].size, 72), p[0].reshape(-1))
    np.testing.assert_array_equal(np.frombuffer(buf, "<f4", p[0].size, 72 + 4 * p[0].size), m[0].reshape(-1))


def test_weights_only_format_resumes_at_step_zero():
    p = _tensors(4)
    buf = ck.encode_weights(CFG, p)
    assert buf[:8] == b"ASCA2CK1" and len(buf) == 56 + sum(8 + 4 * a.size for a in p)
    cfg, step, p2, m2, v2 = ck.decode(buf, ck.model_shapes)
    assert cfg == CFG and step == 0
    for a, b in zip(p, p2):
        np.testing.assert_array_equal(a, b)
    assert all(not x.any() for x in m2 + v2)
    with pytest.raises(ck.CheckpointError):
        ck.peek(buf)   # no step in a weights-only file


def test_truncated_and_foreign_files_are_errors():
    buf = ck.encode_resume(CFG, 7, _tensors(5), _tensors(6), _tensors(7))
    for cut in (0, 5, 8, 40, 63, 64, 70, 1000, len(buf) - 1):
        with pytest.raises(ck.CheckpointError):
            ck.decode(buf[:cut], ck.model_shapes)
    with pytest.raises(ck.CheckpointError):
        ck.decode(b"NOTASCA!" + buf[8:], ck.model_shapes)
    # a count that disagrees with the config's tensor
    bad = bytearray(buf)
    struct.pack_into("<Q", bad, 64, 3)
    with pytest.raises(ck.CheckpointError):
        ck.decode(bytes(bad), ck.model_shapes)


def test_atomic_write_leaves_no_temporary(tmp_path):
    path = str(tmp_path / "model.ck")
    ck.write_atomic(path, b"old")
    ck.write_atomic(path, ck.encode_weights(CFG, _tensors(8)))
    assert open(path, "rb").read(8) == b"ASCA2CK1"
    assert not os.path.exists(path + ".tmp")
