"""Pins of the chunked-form restatement (oracle/chunked_oracle.py).

* Recurrent == chunked (docs/SPEC_V2.md:63 claims agreement to 1.8e-15 in
  fp64 for chunks 8/16/40/64): the float64 chunked forward against a float64
  recurrence written from the equations, for several chunk sizes including a
  ragged last chunk, to 1e-12.
* Its backward against float64 torch autograd of that recurrence, to 1e-10,
  with gates pushed towards 0 and 1 so a dropped decay term shows.
* Against the C oracle (the reference's scan_cpu / bptt_cpu restatement) on
  the configs' input distributions, to the parity bars.
"""
import numpy as np
import pytest
import torch

from oracle import chunked_oracle as co


def _recurrent_torch(q, k, v, a, b, B, T, H, dh):
    o = torch.zeros(B, H, T, dh, dtype=torch.float64)
    outs = []
    for bb in range(B):
        for h in range(H):
            S = torch.zeros(dh, dh, dtype=torch.float64)
            rows = []
            for t in range(T):
                r = bb * T + t
                kt, qt, vt = k[r, h * dh:(h + 1) * dh], q[r, h * dh:(h + 1) * dh], v[r, h * dh:(h + 1) * dh]
                al, be = a[r, h], b[r, h]
                sk = S.T @ kt
                u = be * (vt - al * sk)
                S = al * S + torch.outer(kt, u)
                rows.append(S.T @ qt)
            outs.append(torch.stack(rows))
    o = torch.stack(outs).reshape(B, H, T, dh)
    return o.permute(0, 2, 1, 3).reshape(B * T, H * dh)


def _inputs(seed, B, T, H, dh, spread=1.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B * T, H * dh))
    k = rng.standard_normal((B * T, H * dh))
    for x in (q, k):
        x3 = x.reshape(B * T, H, dh)
        x3 /= np.linalg.norm(x3, axis=2, keepdims=True)
    v = rng.standard_normal((B * T, H * dh))
    a = 1 / (1 + np.exp(-(2 + spread * rng.standard_normal((B * T, H)))))
    b = 1 / (1 + np.exp(-spread * rng.standard_normal((B * T, H))))
    d_o = rng.standard_normal((B * T, H * dh))
    return q, k, v, a, b, d_o


@pytest.mark.parametrize("C", [8, 16, 40, 64])
def test_chunked_equals_recurrent_float64(C):
    B, T, H, dh = 2, 100, 2, 16
    q, k, v, a, b, d_o = _inputs(C, B, T, H, dh, spread=3.0)
    o, cache = co.fwd(q, k, v, a, b, B, T, H, dh, C)
    t = [torch.tensor(x, requires_grad=True) for x in (q, k, v, a, b)]
    o_ref = _recurrent_torch(*t, B, T, H, dh)
    assert np.max(np.abs(o - o_ref.detach().numpy())) <= 1e-12 * np.max(np.abs(o))
    (o_ref * torch.tensor(d_o)).sum().backward()
    grads = co.bwd(cache, d_o)
    for name, g, ref in zip(("dq", "dk", "dv", "dalpha", "dbeta"), grads, t):
        r = ref.grad.numpy()
        assert np.max(np.abs(g - r)) <= 1e-10 * np.max(np.abs(r)), name


def test_chunked_against_the_c_oracle(orc):
    B, T, H, dh = 2, 130, 2, 32
    x = orc.DeltaInputs(3, B, T, H, dh)
    o_ref, dq, dk, dv, da, db = orc.delta_fwd_bwd(x.q, x.k, x.v, x.alpha, x.beta, x.d_o, B, T, H, dh)
    o, cache = co.fwd(x.q, x.k, x.v, x.alpha, x.beta, B, T, H, dh, 64)
    assert orc.rel_err(o, o_ref) <= 2e-6
    for g, ref in zip(co.bwd(cache, x.d_o), (dq, dk, dv, da, db)):
        assert orc.rel_err(g, ref) <= 1e-5


def test_chunked_dalpha_at_zero_and_tiny_gates():
    # dalpha from products with alpha_m left out (no division): finite at
    # alpha = 0 and equal to autograd of the recurrence there
    B, T, H, dh, C = 1, 48, 2, 8, 16
    q, k, v, a, b, d_o = _inputs(5, B, T, H, dh)
    t = np.arange(T)
    a[t % 7 == 3] = 0.0
    a[(t >= 20) & (t < 30), 0] = 1e-6
    a[(t >= 32) & (t < 36), 1] = 1.5
    o, cache = co.fwd(q, k, v, a, b, B, T, H, dh, C)
    tt = [torch.tensor(x, requires_grad=True) for x in (q, k, v, a, b)]
    o_ref = _recurrent_torch(*tt, B, T, H, dh)
    (o_ref * torch.tensor(d_o)).sum().backward()
    grads = co.bwd(cache, d_o)
    assert all(np.isfinite(gr).all() for gr in grads)
    for name, gr, ref in zip(("dq", "dk", "dv", "dalpha", "dbeta"), grads, tt):
        r = ref.grad.numpy()
        assert np.max(np.abs(gr - r)) <= 1e-10 * np.max(np.abs(r)), name
