"""GPU parity of the device-resident training step (asca_model_* via
asca_amd.model.DeviceModel) against the model oracle (oracle/model_oracle.py),
on identical parameters and tokens.

Bars: the loss (a forward quantity) <= 2e-5 relative, every gradient tensor
<= 1e-4 as max|gpu-cpu|/max|cpu| (rust/src/main.rs:1021-1029); the AdamW step
over all tensors bit-exact given the same gradients.
"""
import numpy as np
import pytest

from oracle import model_oracle as mo

pytestmark = pytest.mark.gpu

FWD_TOL = 2e-5
GRAD_TOL = 1e-4


def _models(cfg, seed):
    from asca_amd.model import DeviceModel

    V, d, H, L, E, dff = cfg
    p = mo.init_params(seed, V, d, H, L, E, dff)
    dm = DeviceModel(V, d, H, L, E, dff)
    dm.set_params(p)
    return dm, mo.OracleModel(V, d, H, L, E, dff, [a.copy() for a in p])


@pytest.mark.parametrize("cfg,batch,seq", [
    ((256, 16, 2, 1, 2, 16), 1, 10),        # the reference's gradcheck_model shape
    ((256, 64, 4, 2, 8, 128), 2, 32),
    ((256, 512, 8, 1, 16, 1024), 2, 64),    # configs[3] widths, 128 tokens
    ((256, 512, 8, 8, 16, 1024), 1, 1024),  # configs[3] at full depth and length, one of its 16 sequences
    ((200, 48, 3, 2, 5, 40), 3, 17),        # ragged: odd widths, dh 16, T not a multiple of 8
    ((256, 128, 4, 1, 4, 64), 3, 100),      # gate projection on the 16-column kernels with K = 128, 300 rows
    ((256, 256, 16, 1, 4, 64), 2, 20),      # 2H = 32 gate columns: the general GEMM
])
def test_train_step_grads_match_oracle(cfg, batch, seq):
    dm, om = _models(cfg, 21)
    rng = np.random.default_rng(sum(cfg) + batch * seq)
    n = batch * seq
    ids = rng.integers(0, cfg[0], n).astype(np.uint32)
    tgts = rng.integers(0, cfg[0], n).astype(np.uint32)
    print(f"[model] cfg={cfg} batch={batch} seq={seq}", flush=True)
    loss = dm.forward_backward(ids, tgts, batch)
    rloss, rgrads = om.forward_backward(ids, tgts, batch)
    print(f"[model]   loss gpu {loss:.7f} cpu {rloss:.7f}", flush=True)
    assert abs(loss - rloss) <= FWD_TOL * abs(rloss)
    names = mo.tensor_names(cfg[3])
    worst = 0.0
    for name, got, want in zip(names, dm.grads(), rgrads):
        err = 0.0 if np.max(np.abs(want)) == 0 and np.max(np.abs(got)) == 0 else \
            np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30)
        worst = max(worst, err)
        assert err <= GRAD_TOL, (name, err)
    print(f"[model]   worst grad rel err {worst:.2e}", flush=True)
    dm.close()


@pytest.mark.parametrize("cfg", [
    (256, 64, 4, 2, 8, 128),
    (255, 48, 3, 1, 3, 40),   # tensors whose sizes are not multiples of 4 (b_gate: 6)
])
def test_adamw_over_all_tensors_bit_exact(cfg):
    dm, om = _models(cfg, 5)
    rng = np.random.default_rng(2)
    grads = [rng.standard_normal(a.shape).astype(np.float32) for a in om.p]
    m = [(0.01 * rng.standard_normal(a.shape)).astype(np.float32) for a in om.p]
    v = [(0.01 * np.abs(rng.standard_normal(a.shape))).astype(np.float32) for a in om.p]
    dm.set_grads(grads)
    dm.set_moments(m, v)
    dm.set_adamw(3e-4, 0.9, 0.95, 1e-8, 0.01, step=37)
    dm.adamw()
    step = om.adamw(grads, m, v, 37)
    assert dm.adamw_step_count() == step == 37 + len(om.p)
    gm, gv = dm.moments()
    for name, a, b in zip(mo.tensor_names(cfg[3]), dm.params(), om.p):
        np.testing.assert_array_equal(a, b, err_msg=name)
    for a, b in zip(gm, m):
        np.testing.assert_array_equal(a, b)
    for a, b in zip(gv, v):
        np.testing.assert_array_equal(a, b)
    dm.close()


def test_two_train_steps_follow_the_oracle():
    cfg = (256, 64, 4, 2, 8, 128)
    dm, om = _models(cfg, 8)
    rng = np.random.default_rng(3)
    ids = rng.integers(0, 256, 64).astype(np.uint32)
    tgts = rng.integers(0, 256, 64).astype(np.uint32)
    dm.set_adamw()
    mm = [np.zeros_like(a) for a in om.p]
    vv = [np.zeros_like(a) for a in om.p]
    step = 0
    for it in range(2):
        loss = dm.train_step(ids, tgts, 2)
        rloss, g = om.forward_backward(ids, tgts, 2)
        step = om.adamw(g, mm, vv, step)
        print(f"[model] step {it}: loss gpu {loss:.7f} cpu {rloss:.7f}", flush=True)
        assert abs(loss - rloss) <= FWD_TOL * abs(rloss)
    # the loss after the two updates, evaluated by both sides
    loss2 = dm.forward_backward(ids, tgts, 2)
    rloss2, _ = om.forward_backward(ids, tgts, 2)
    assert abs(loss2 - rloss2) <= 1e-4 * abs(rloss2)
    assert rloss2 < rloss
    dm.close()


def test_train_step_equals_backward_then_adamw():
    """asca_model_train_step applies AdamW per layer during the backward (on the
    model's second stream); the parameters and moments must be bit-identical to
    a forward_backward followed by one AdamW launch over all tensors."""
    cfg = (256, 512, 8, 2, 16, 1024)
    a, _ = _models(cfg, 31)
    b, _ = _models(cfg, 31)
    rng = np.random.default_rng(4)
    for dm in (a, b):
        dm.set_adamw(step=5)
    for it in range(2):
        ids = rng.integers(0, 256, 3 * 40).astype(np.uint32)
        tgts = rng.integers(0, 256, 3 * 40).astype(np.uint32)
        la = a.train_step(ids, tgts, 3)
        lb = b.forward_backward(ids, tgts, 3)
        b.adamw()
        assert la == lb
    assert a.adamw_step_count() == b.adamw_step_count() == 5 + 2 * len(a.params())
    for x, y in zip(a.params(), b.params()):
        np.testing.assert_array_equal(x, y)
    for ma, mb in zip(a.moments(), b.moments()):
        for x, y in zip(ma, mb):
            np.testing.assert_array_equal(x, y)
    a.close()
    b.close()


def test_config3_full_step_runs_deterministically():
    """configs[3] at full size (V=256, d=512, 8 layers, H=8, E=16, d_ff=1024,
    B=16, T=1024): a forward+backward from N(0, 0.02) weights gives a finite
    loss near ln(256) and bit-identical gradients on a rerun."""
    from asca_amd.model import DeviceModel

    V, d, H, L, E, dff = 256, 512, 8, 8, 16, 1024
    dm = DeviceModel(V, d, H, L, E, dff)
    rng = np.random.default_rng(2)
    dm.set_params([(0.02 * rng.standard_normal((r, c))).astype(np.float32) for _, _, r, c in dm.tensors])
    ids = rng.integers(0, 256, 16 * 1024).astype(np.uint32)
    tgts = np.roll(ids, -1)
    print("[model] configs[3] full step", flush=True)
    l1 = dm.forward_backward(ids, tgts, 16)
    g1 = dm.grads()
    l2 = dm.forward_backward(ids, tgts, 16)
    g2 = dm.grads()
    print(f"[model]   loss {l1:.6f}", flush=True)
    assert np.isfinite(l1) and abs(l1 - np.log(256)) < 0.5
    assert l1 == l2
    for a, b in zip(g1, g2):
        np.testing.assert_array_equal(a, b)
    dm.close()


@pytest.mark.parametrize("cfg,batch,seq", [
    ((256, 64, 4, 2, 8, 128), 1, 24),       # the reference's decode gate: Config::tiny, 24 tokens
    ((256, 64, 4, 2, 8, 128), 5, 13),       # several sequences per step
    ((256, 512, 8, 1, 16, 1024), 3, 9),     # configs[3] widths (dh 64)
    ((200, 48, 3, 2, 5, 40), 2, 11),        # odd widths, dh 16
])
def test_decode_steps_match_forward(cfg, batch, seq):
    # rust/tests/decode_parity.rs: decoding token by token on carried states
    # gives the logits of one full forward over the sequence, within 1e-4 of
    # the largest logit (decode_parity.rs:36); here against the oracle forward.
    V = cfg[0]
    dm, om = _models(cfg, 17)
    rng = np.random.default_rng(3 + batch * seq)
    ids = rng.integers(0, V, (batch, seq)).astype(np.uint32)
    print(f"[decode] cfg={cfg} batch={batch} seq={seq}", flush=True)
    ref, _ = om.forward(ids.reshape(-1), batch)
    ref = ref.reshape(batch, seq, V)
    st = dm.new_decode_state(batch)
    worst = 0.0
    for t in range(seq):
        got = dm.step(ids[:, t], st)
        worst = max(worst, float(np.max(np.abs(got - ref[:, t]))))
    rel = worst / float(np.max(np.abs(ref)))
    print(f"[decode]   worst |dlogit| {worst:.3e}, relative {rel:.3e}", flush=True)
    assert rel <= 1e-4
    # the states hold exactly L * H * dh^2 floats per sequence, whatever the length
    assert dm.decode_state_floats() == cfg[3] * cfg[1] * (cfg[1] // cfg[2])
    dm.close()


def test_checkpoint_resume_round_trip(tmp_path):
    # train.rs:303-455 on the device-resident model: save_resume writes the
    # weights and the moments held in HBM; load_resume restores them bit for
    # bit with the AdamW counter at the saved step, and training continues
    # exactly as on the original model given the same counter.
    from asca_amd import checkpoint as ck

    cfg = (256, 64, 4, 2, 8, 128)
    dm, _ = _models(cfg, 9)
    rng = np.random.default_rng(9)
    ids = rng.integers(0, 256, 48).astype(np.uint32)
    tgt = rng.integers(0, 256, 48).astype(np.uint32)
    dm.train_step(ids, tgt, 2)
    dm.train_step(ids, tgt, 2)
    path = str(tmp_path / "resume.ck")
    ck.save_resume(path, dm, 2)
    assert ck.peek_resume(path) == (cfg, 2)
    dm2, step = ck.load_resume(path)
    assert step == 2 and dm2.adamw_step_count() == 2
    for a, b in zip(dm.params(), dm2.params()):
        np.testing.assert_array_equal(a, b)
    for x, y in zip(dm.moments(), dm2.moments()):
        for a, b in zip(x, y):
            np.testing.assert_array_equal(a, b)
    dm.set_adamw(step=2)
    l1 = dm.train_step(ids, tgt, 2)
    l2 = dm2.train_step(ids, tgt, 2)
    assert l1 == l2
    for a, b in zip(dm.params(), dm2.params()):
        np.testing.assert_array_equal(a, b)
    # weights-only file: same weights, zero moments
    wpath = str(tmp_path / "weights.ck")
    ck.save(wpath, dm)
    dm3 = ck.load(wpath)
    for a, b in zip(dm.params(), dm3.params()):
        np.testing.assert_array_equal(a, b)
    assert all(not a.any() for a in dm3.moments()[0])
    for x in (dm, dm2, dm3):
        x.close()


def _launches():
    import ctypes as C
    from asca_amd import _lib

    h2d, d2h, n = C.c_uint64(), C.c_uint64(), C.c_uint64()
    _lib.call("asca_stats", C.byref(h2d), C.byref(d2h), C.byref(n))
    return n.value


@pytest.mark.parametrize("where", ["forward", "mid-backward", "last backward launch", "optimiser"])
def test_train_step_failure_leaves_parameters_untouched(where):
    """A launch that fails inside the forward or backward makes
    asca_model_train_step return the error with the parameters, AdamW moments
    and step count exactly as before, and the caller's repeat of the step gives
    what a model that never failed gets.  A failure among the optimiser's
    launches (queued only after the whole backward) is ASCA_ERR_PARTIAL_UPDATE:
    the groups queued before it moved, the step count did not."""
    from asca_amd import gpu
    from asca_amd._lib import AscaError

    cfg = (256, 64, 4, 2, 4, 64)
    L = cfg[3]
    a, _ = _models(cfg, 41)
    b, _ = _models(cfg, 41)
    rng = np.random.default_rng(9)
    ids = rng.integers(0, 256, 2 * 24).astype(np.uint32)
    tgts = rng.integers(0, 256, 2 * 24).astype(np.uint32)
    a.train_step(ids, tgts, 2)
    n0 = _launches()
    b.train_step(ids, tgts, 2)
    per_step = _launches() - n0
    n_opt = L + 2                       # head, each layer, embedding
    fail_at = {"forward": 3, "mid-backward": (per_step - n_opt) * 3 // 4,
               "last backward launch": per_step - n_opt - 1, "optimiser": per_step - 2}[where]
    p0, m0, s0 = a.params(), a.moments(), a.adamw_step_count()
    print(f"[model] {per_step} launches per step; injected failure at launch {fail_at} ({where})", flush=True)
    gpu.fail_after(fail_at)
    with pytest.raises(AscaError) as ei:
        a.train_step(ids, tgts, 2)
    gpu.fail_after(-1)
    assert a.adamw_step_count() == s0
    p1, m1 = a.params(), a.moments()
    if where == "optimiser":
        assert ei.value.code == 8, ei.value
        # the groups before the failing one (all but the embedding, tensor 0) moved
        assert np.array_equal(p1[0], p0[0]) and not np.array_equal(p1[1], p0[1])
        a.close()
        b.close()
        return
    assert ei.value.code == 5, ei.value
    for x, y in zip(p1, p0):
        np.testing.assert_array_equal(x, y)
    for ma, mb in zip(m1, m0):
        for x, y in zip(ma, mb):
            np.testing.assert_array_equal(x, y)
    la = a.train_step(ids, tgts, 2)
    lb = b.train_step(ids, tgts, 2)
    assert la == lb
    for x, y in zip(a.params(), b.params()):
        np.testing.assert_array_equal(x, y)
    a.close()
    b.close()


def test_device_batch_parity():
    """rust/tests/batch_parity.rs:20-133 on the device: one training step on a
    batch of 4 sequences of 12 tokens equals the mean of four single-sequence
    steps (loss within 1e-5, every gradient within 2e-4 relative, the
    reference's bars), with Config::tiny (rust/src/model.rs:32-41) and the
    reference's seeds (Rng(5) for ids and targets below 256, Rng(9) for the
    parameters)."""
    import ctypes as C
    from asca_amd import _lib

    cfg, batch, seq = (256, 64, 4, 2, 8, 128), 4, 12
    dm, _ = _models(cfg, 9)
    st = (C.c_uint64 * 2)()
    lib = _lib.load()
    lib.asca_rng_seed(5, st)
    raw = np.empty(2 * batch * seq, np.uint64)
    lib.asca_rng_u64(st, raw.ctypes.data_as(C.POINTER(C.c_uint64)), raw.size)
    ids = (raw[:batch * seq] % np.uint64(256)).astype(np.uint32)
    tgts = (raw[batch * seq:] % np.uint64(256)).astype(np.uint32)
    loss1, acc = 0.0, None
    for b in range(batch):
        s = slice(b * seq, (b + 1) * seq)
        loss1 += dm.forward_backward(ids[s], tgts[s], 1)
        gr = [g.astype(np.float64) for g in dm.grads()]
        acc = gr if acc is None else [a + g for a, g in zip(acc, gr)]
    loss1 /= batch
    g1 = [(a / batch).astype(np.float32) for a in acc]
    lossb = dm.forward_backward(ids, tgts, batch)
    gb = dm.grads()
    rel = abs(loss1 - lossb) / max(abs(loss1), abs(lossb), 1e-6)
    worst = 0.0
    for name, a, b in zip(mo.tensor_names(cfg[3]), g1, gb):
        err = np.max(np.abs(a - b)) / max(np.max(np.abs(a)), 1e-9)
        worst = max(worst, err)
        assert err <= 2e-4, (name, err)
    print(f"[model] device batch parity: loss batch=1 {loss1:.6f} batch=4 {lossb:.6f} (rel {rel:.2e}), "
          f"worst grad rel {worst:.2e}", flush=True)
    assert rel <= 1e-5
    dm.close()
