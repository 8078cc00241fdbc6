"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the restatement (a dropped
term, a swapped index, a sign) fails one of them:
  * golden vectors from independent implementations (tests/golden/make_golden.py):
    integer Rng streams, integer hash routing, float64 torch autograd of the
    delta rule in matrix form, float64 decode steps;
  * closed forms of the recurrence;
  * central finite differences (restating rust/tests/gradcheck.rs:43-49);
  * the reference's invariants: batch isolation (rust/src/main.rs:954-981,
    rust/tests/batch_parity.rs) and decode == forward (rust/tests/decode_parity.rs).
"""
import json

import numpy as np
import pytest

from conftest import GOLDEN


def test_rng_u64_matches_integer_golden(orc):
    gold = json.loads((GOLDEN / "rng.json").read_text())
    for seed, vals in gold["u64"].items():
        got = orc.rng_u64(int(seed), len(vals))
        assert [int(x) for x in got] == [int(v) for v in vals], seed


def test_rng_normal_matches_float64_box_muller(orc):
    gold = json.loads((GOLDEN / "rng.json").read_text())
    for seed, vals in gold["normal_f64"].items():
        got = orc.rng_normal(int(seed), len(vals)).astype(np.float64)
        # f32 logf/cosf/sqrtf against float64: a few ulp
        np.testing.assert_allclose(got, np.array(vals), rtol=2e-6, atol=2e-6)


def test_hash_route_golden_and_survey_fixture(orc):
    gold = json.loads((GOLDEN / "hash.json").read_text())
    ids = np.arange(4096, dtype=np.uint32)
    for n, vals in gold.items():
        assert orc.hash_route(ids, int(n)).tolist() == vals
    r = orc.hash_route(np.arange(16), 16).tolist()
    assert r == [0, 4, 5, 14, 5, 8, 1, 15, 11, 5, 12, 3, 2, 4, 6, 3]
    counts = np.bincount(orc.hash_route(np.arange(256), 16), minlength=16).tolist()
    assert counts == [14, 20, 19, 17, 14, 18, 18, 20, 15, 15, 12, 19, 15, 13, 10, 17]


def _tiny():
    z = np.load(GOLDEN / "delta_tiny.npz")
    return {k: z[k] for k in z.files}


def test_scan_and_raw_bptt_match_autograd_golden(orc):
    z = _tiny()
    B, T, H, dh = int(z["B"]), int(z["T"]), int(z["H"]), int(z["dh"])
    o, st = orc.delta_scan(z["q"], z["k"], z["v"], z["alpha"], z["beta"], B, T, H, dh)
    assert orc.rel_err(o, z["o"]) < 2e-6
    # final state of unit (h*B + b) against the float64 S_T[b, h]
    for h in range(H):
        for b in range(B):
            s_last = st[h * B + b, T * dh * dh:].reshape(dh, dh)
            assert orc.rel_err(s_last, z["s_final"][b, h]) < 2e-6
    g = orc.delta_bptt_raw(z["q"], z["k"], z["v"], z["alpha"], z["beta"], z["d_o"], st, B, T, H, dh)
    for name, got in zip(("dq", "dk", "dv", "dalpha", "dbeta"), g):
        assert orc.rel_err(got, z[name]) < 1e-5, name


def test_fused_grads_match_autograd_through_norm_and_sigmoid(orc):
    z = _tiny()
    B, T, H, dh = int(z["B"]), int(z["T"]), int(z["H"]), int(z["dh"])
    q, qn = orc.l2norm_heads(z["q_raw"], H, dh)
    k, kn = orc.l2norm_heads(z["k_raw"], H, dh)
    alpha = (1.0 / (1.0 + np.exp(-z["gate_a"].astype(np.float32)))).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-z["gate_b"].astype(np.float32)))).astype(np.float32)
    o, st = orc.delta_scan(q, k, z["v"], alpha, beta, B, T, H, dh)
    raw = orc.delta_bptt_raw(q, k, z["v"], alpha, beta, z["d_o"], st, B, T, H, dh)
    d_qkv, d_gate = orc.delta_fuse(q, k, qn, kn, alpha, beta, *raw, H, dh)
    assert orc.rel_err(d_qkv, z["d_qkv"]) < 1e-5
    assert orc.rel_err(d_gate, z["d_gate"]) < 1e-5


def _inputs(orc, seed, B, T, H, dh):
    return orc.DeltaInputs(seed, B, T, H, dh)


def test_closed_form_no_write(orc):
    # alpha = 1, beta = 0: S stays 0, o = 0
    x = _inputs(orc, 3, 2, 9, 2, 8)
    o, st = orc.delta_scan(x.q, x.k, x.v, np.ones_like(x.alpha), np.zeros_like(x.beta), 2, 9, 2, 8)
    assert np.all(o == 0) and np.all(st == 0)


def test_closed_form_orthonormal_keys_recall_values(orc):
    # k_t = e_t, alpha = 1, beta = 1, q_t = k_t: S^T e_j = v_j so o_t = v_t
    T = dh = 8
    H, B = 1, 1
    k = np.eye(T, dtype=np.float32)
    v = np.random.default_rng(0).standard_normal((T, dh)).astype(np.float32)
    ones = np.ones((T, 1), dtype=np.float32)
    o, _ = orc.delta_scan(k.copy(), k, v, ones, ones, B, T, H, dh)
    np.testing.assert_array_equal(o, v)


def test_invariant_beta_one_writes_value(orc):
    # beta = 1, |k| = 1: S_t^T k_t = alpha(1-beta) S_{t-1}^T k_t + beta v_t = v_t
    B, T, H, dh = 2, 64, 2, 16
    x = _inputs(orc, 5, B, T, H, dh)
    beta = np.ones_like(x.beta)
    _, st = orc.delta_scan(x.q, x.k, x.v, x.alpha, beta, B, T, H, dh)
    worst = 0.0
    for h in range(H):
        for b in range(B):
            for t in range(T):
                S = st[h * B + b, (t + 1) * dh * dh:(t + 2) * dh * dh].reshape(dh, dh)
                r = b * T + t
                kt = x.k[r, h * dh:(h + 1) * dh]
                vt = x.v[r, h * dh:(h + 1) * dh]
                worst = max(worst, float(np.max(np.abs(S.T @ kt - vt))))
    assert worst < 1e-5


def test_closed_form_single_step(orc):
    # from S_0 = 0, one step gives o = beta (q . k) v
    x = _inputs(orc, 9, 3, 1, 2, 16)
    o, _ = orc.delta_scan(x.q, x.k, x.v, x.alpha, x.beta, 3, 1, 2, 16)
    for r in range(3):
        for h in range(2):
            sl = slice(h * 16, (h + 1) * 16)
            want = x.beta[r, h] * np.dot(x.q[r, sl].astype(np.float64), x.k[r, sl]) * x.v[r, sl]
            np.testing.assert_allclose(o[r, sl], want, rtol=1e-5, atol=1e-6)


def test_batch_isolation_bit_exact(orc):
    # rust/src/main.rs:954-981: batch B equals B separate batch-1 scans, bitwise
    B, T, H, dh = 3, 24, 4, 16
    x = _inputs(orc, 21, B, T, H, dh)
    o, st = orc.delta_scan(x.q, x.k, x.v, x.alpha, x.beta, B, T, H, dh)
    g = orc.delta_bptt_raw(x.q, x.k, x.v, x.alpha, x.beta, x.d_o, st, B, T, H, dh)
    for b in range(B):
        rs = slice(b * T, (b + 1) * T)
        sub = [np.ascontiguousarray(a[rs]) for a in (x.q, x.k, x.v, x.alpha, x.beta, x.d_o)]
        o1, st1 = orc.delta_scan(*sub[:5], 1, T, H, dh)
        g1 = orc.delta_bptt_raw(*sub, st1, 1, T, H, dh)
        np.testing.assert_array_equal(o1, o[rs])
        for a, a1 in zip(g, g1):
            np.testing.assert_array_equal(a1, a[rs])


def test_finite_differences_raw_grads(orc):
    # rust/tests/gradcheck.rs:25-58 tolerance: 2e-2*max(|a|,|n|) + 1e-3*max|grad|,
    # here on the recurrence inputs with L = sum(o * dO), float32, eps = 1e-3
    B, T, H, dh = 1, 12, 2, 8
    x = _inputs(orc, 7, B, T, H, dh)
    args = [x.q, x.k, x.v, x.alpha, x.beta]
    o, st = orc.delta_scan(*args, B, T, H, dh)
    grads = orc.delta_bptt_raw(*args, x.d_o, st, B, T, H, dh)

    def loss(a):
        oo, _ = orc.delta_scan(*a, B, T, H, dh, with_states=False)
        return float(np.sum(oo.astype(np.float64) * x.d_o))

    eps = 1e-3
    fails = []
    for idx, (arr, gr) in enumerate(zip(args, grads)):
        scale = max(float(np.max(np.abs(gr))), 1e-3)
        flat = arr.reshape(-1)
        for i in range(0, flat.size, max(flat.size // 23, 1)):
            a_p = [a.copy() for a in args]
            a_m = [a.copy() for a in args]
            a_p[idx].reshape(-1)[i] += eps
            a_m[idx].reshape(-1)[i] -= eps
            num = (loss(a_p) - loss(a_m)) / (2 * eps)
            ana = float(gr.reshape(-1)[i])
            tol = 2e-2 * max(abs(ana), abs(num)) + 1e-3 * scale
            if abs(ana - num) > tol:
                fails.append((idx, i, ana, num))
    assert not fails, fails[:5]


def test_decode_step_matches_float64_golden(orc):
    z = np.load(GOLDEN / "decode_tiny.npz")
    n_seq, H, dh = int(z["n_seq"]), int(z["H"]), int(z["dh"])
    S = np.zeros((n_seq, H, dh, dh), dtype=np.float32)
    for s in range(z["qkv"].shape[0]):
        o = orc.delta_decode_step(S, np.ascontiguousarray(z["qkv"][s]), np.ascontiguousarray(z["gate"][s]), H, dh)
        assert orc.rel_err(o, z["o"][s]) < 2e-6
    assert orc.rel_err(S, z["s_final"]) < 2e-6


def test_decode_equals_forward(orc):
    # rust/tests/decode_parity.rs: token-by-token step == full forward, rel <= 1e-4
    T, H, dh = 20, 2, 16
    d = H * dh
    rng = np.random.default_rng(4)
    qkv = rng.standard_normal((T, 3 * d)).astype(np.float32)
    gate = rng.standard_normal((T, 2 * H)).astype(np.float32)
    gate[:, :H] += 2
    q, _ = orc.l2norm_heads(qkv[:, :d], H, dh)
    k, _ = orc.l2norm_heads(qkv[:, d:2 * d], H, dh)
    v = np.ascontiguousarray(qkv[:, 2 * d:])
    a = (1 / (1 + np.exp(-gate[:, :H]))).astype(np.float32)
    b = (1 / (1 + np.exp(-gate[:, H:]))).astype(np.float32)
    o_fwd, _ = orc.delta_scan(q, k, v, a, b, 1, T, H, dh)
    S = np.zeros((1, H, dh, dh), dtype=np.float32)
    o_dec = np.stack([orc.delta_decode_step(S, qkv[t:t + 1].copy(), gate[t:t + 1].copy(), H, dh)[0]
                      for t in range(T)])
    assert orc.rel_err(o_dec, o_fwd) < 1e-4


def test_rmsnorm_against_float64(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((37, 203)).astype(np.float32)
    dy = rng.standard_normal((37, 203)).astype(np.float32)
    x64, dy64 = x.astype(np.float64), dy.astype(np.float64)
    inv = 1 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-6)
    assert orc.rel_err(orc.rmsnorm(x), x64 * inv) < 2e-6
    xh = x64 * inv
    dx = inv * (dy64 - xh * (dy64 * xh).mean(1, keepdims=True))
    assert orc.rel_err(orc.rmsnorm_bwd(x, dy), dx) < 2e-6


def test_adamw_against_float64_and_step_counter(orc):
    rng = np.random.default_rng(2)
    p = rng.standard_normal(1000).astype(np.float32)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    p64, m64, v64 = p.astype(np.float64), m.astype(np.float64), v.astype(np.float64)
    step = 0
    for it in range(5):
        gr = rng.standard_normal(1000).astype(np.float32)
        step = orc.adamw(p, gr, m, v, 3e-4, step)
        # rust/src/tensor.rs:392-402,444-453: lr*sqrt(bc1/bc2), eps*sqrt(bc2), wd = lr*0.01
        bc1, bc2 = 1 - 0.9 ** step, 1 - 0.95 ** step
        m64 = 0.9 * m64 + 0.1 * gr
        v64 = 0.95 * v64 + 0.05 * gr.astype(np.float64) ** 2
        upd = m64 / (np.sqrt(v64) + 1e-8 * np.sqrt(bc2))
        p64 = p64 - 3e-4 * 0.01 * p64
        p64 = p64 - 3e-4 * np.sqrt(bc1 / bc2) * upd
        assert step == it + 1
        assert np.max(np.abs(p - p64)) < 1e-6
