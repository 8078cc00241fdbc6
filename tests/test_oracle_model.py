"""Pins of the model-level oracle (oracle/model_oracle.py).

* Finite differences over every tensor, restating the reference's own model
  check rust/tests/gradcheck_model.rs (V=256, d=16, H=2, L=1, E=2, d_ff=16,
  10 tokens; eps=3e-4; the 4 largest-gradient entries per tensor; tolerance
  5% + the f32 noise floor; entries under the noise floor skipped).
* Batch isolation of the forward (rust/tests/batch_parity.rs): a batch of B
  sequences gives the logits of B separate batch-1 forwards.
* The AdamW step counter advancing once per tensor (tensor.rs:393): tensor j
  of the first optimiser step is updated with bias corrections of step j+1,
  checked against a float64 evaluation of the closed-form first update.
"""
import numpy as np

from oracle import model_oracle as mo


def _tiny(seed=11):
    V, d, H, L, E, dff = 256, 16, 2, 1, 2, 16
    p = mo.init_params(seed, V, d, H, L, E, dff)
    return mo.OracleModel(V, d, H, L, E, dff, p)


def test_model_oracle_finite_differences(orc):
    m = _tiny()
    rng = np.random.default_rng(11)
    ids = rng.integers(0, 256, 10).astype(np.uint32)
    tgts = rng.integers(0, 256, 10).astype(np.uint32)
    loss, grads = m.forward_backward(ids, tgts, 1)
    assert abs(loss - m.loss(ids, tgts)) <= 1e-6 * abs(loss)
    eps = np.float32(3e-4)
    ulp = max(abs(loss), 1.0) * np.finfo(np.float32).eps
    noise = 4.0 * ulp / (2.0 * eps)
    checked = 0
    for i, name in enumerate(mo.tensor_names(1)):
        g = grads[i].reshape(-1)
        for j in np.argsort(-np.abs(g), kind="stable")[:4]:
            flat = m.p[i].reshape(-1)
            orig = flat[j]
            flat[j] = orig + eps
            lp = m.loss(ids, tgts)
            flat[j] = orig - eps
            lm = m.loss(ids, tgts)
            flat[j] = orig
            numeric = (lp - lm) / (2.0 * eps)
            analytic = float(g[j])
            if abs(analytic) < 3.0 * noise:
                continue
            tol = 0.05 * abs(analytic) + noise
            assert abs(analytic - numeric) <= tol, (name, j, analytic, numeric)
            checked += 1
    assert checked >= 20


def test_model_oracle_batch_isolation():
    V, d, H, L, E, dff = 256, 32, 4, 2, 4, 32
    m = mo.OracleModel(V, d, H, L, E, dff, mo.init_params(3, V, d, H, L, E, dff))
    rng = np.random.default_rng(4)
    ids = rng.integers(0, 256, 3 * 20).astype(np.uint32)
    logits, _ = m.forward(ids, 3)
    for b in range(3):
        lb, _ = m.forward(ids[b * 20:(b + 1) * 20], 1)
        np.testing.assert_allclose(lb, logits[b * 20:(b + 1) * 20], rtol=0, atol=1e-5 * np.abs(logits).max())


def test_model_oracle_adamw_counter_per_tensor():
    V, d, H, L, E, dff = 256, 8, 2, 1, 2, 8
    m = mo.OracleModel(V, d, H, L, E, dff, mo.init_params(5, V, d, H, L, E, dff))
    p0 = [a.copy() for a in m.p]
    rng = np.random.default_rng(6)
    grads = [rng.standard_normal(a.shape).astype(np.float32) for a in m.p]
    mm = [np.zeros_like(a) for a in m.p]
    vv = [np.zeros_like(a) for a in m.p]
    lr, b1, b2, eps, wd = 3e-4, 0.9, 0.95, 1e-8, 0.01
    step = m.adamw(grads, mm, vv, 0, lr, b1, b2, eps, wd)
    assert step == len(m.p)
    for j, (p, g, new) in enumerate(zip(p0, grads, m.p)):
        s = j + 1
        bc1, bc2 = 1 - b1 ** s, 1 - b2 ** s
        g64 = g.astype(np.float64)
        upd = ((1 - b1) * g64) / (np.sqrt((1 - b2) * g64 * g64) + eps * np.sqrt(bc2))
        ref = p.astype(np.float64) * (1 - lr * wd) - lr * np.sqrt(bc1 / bc2) * upd
        np.testing.assert_allclose(new, ref, rtol=1e-5, atol=1e-9)
