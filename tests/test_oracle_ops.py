"""Pins of the oracle's HashMoE, cross-entropy and bucketing restatements.

The MoE forward is checked against a float64 torch evaluation written from the
equations of rust/src/model.rs:187-306 (torch's own matmul and SiLU), and the
hand-ordered MoE backward (model.rs:339-497) against torch autograd of that
forward, so a dropped term, a wrong expert offset or a transposed weight fails.
Cross-entropy is checked against torch.nn.functional.cross_entropy and its
autograd gradient.  Bucketing is checked against the reference's construction
(push every t into buckets[hash(id)], model.rs:190-193).
"""
import numpy as np
import pytest
import torch

FWD_TOL = 2e-5
GRAD_TOL = 1e-4


def _moe_case(seed, T, d, d_ff, E, zero_frac=0.0):
    rng = np.random.default_rng(seed)
    xn = rng.standard_normal((T, d)).astype(np.float32)
    if zero_frac:
        xn[rng.random((T, d)) < zero_frac] = 0.0  # the CPU path skips zero entries
    w1 = (rng.standard_normal((d, E * d_ff)) / np.sqrt(d)).astype(np.float32)
    b1 = (0.1 * rng.standard_normal(E * d_ff)).astype(np.float32)
    w2 = (rng.standard_normal((E * d_ff, d)) / np.sqrt(d_ff)).astype(np.float32)
    b2 = (0.1 * rng.standard_normal(d)).astype(np.float32)
    ids = rng.integers(0, 256, T).astype(np.uint32)
    dout = rng.standard_normal((T, d)).astype(np.float32)
    return xn, w1, b1, w2, b2, ids, dout


def _torch_moe(xn, w1, b1, w2, b2, route, d_ff):
    t = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True)
         for k, v in dict(xn=xn, w1=w1, b1=b1, w2=w2, b2=b2).items()}
    outs, pres = [], []
    for tok in range(xn.shape[0]):
        e = int(route[tok])
        cols = slice(e * d_ff, (e + 1) * d_ff)
        pre = t["xn"][tok] @ t["w1"][:, cols] + t["b1"][cols]
        h = torch.nn.functional.silu(pre)
        outs.append(h @ t["w2"][cols, :] + t["b2"])
        pres.append(pre)
    return t, torch.stack(outs), torch.stack(pres)


@pytest.mark.parametrize("seed,T,d,d_ff,E,zf", [
    (0, 40, 16, 24, 4, 0.0),
    (1, 33, 8, 12, 5, 0.2),   # zero inputs exercise the skip branches
    (2, 17, 12, 8, 1, 0.0),   # one expert
    (3, 9, 8, 8, 16, 0.0),    # more experts than tokens: empty buckets
])
def test_moe_oracle_against_torch_float64(orc, seed, T, d, d_ff, E, zf):
    xn, w1, b1, w2, b2, ids, dout = _moe_case(seed, T, d, d_ff, E, zf)
    route = orc.hash_route(ids, E)
    out, pre, hidden = orc.moe_fwd(xn, w1, b1, w2, b2, route, d_ff)
    t, out_ref, pre_ref = _torch_moe(xn, w1, b1, w2, b2, route, d_ff)
    assert orc.rel_err(out, out_ref.detach().numpy()) <= FWD_TOL
    assert orc.rel_err(pre, pre_ref.detach().numpy()) <= FWD_TOL
    assert orc.rel_err(hidden, torch.nn.functional.silu(pre_ref).detach().numpy()) <= FWD_TOL
    (out_ref * torch.tensor(dout, dtype=torch.float64)).sum().backward()
    dxn, dw1, db1, dw2, db2 = orc.moe_bwd(xn, w1, w2, pre, hidden, route, dout, d_ff)
    for got, name in ((dxn, "xn"), (dw1, "w1"), (db1, "b1"), (dw2, "w2"), (db2, "b2")):
        ref = t[name].grad.numpy()
        assert orc.rel_err(got, ref) <= GRAD_TOL, name


def test_moe_oracle_tokens_are_independent(orc):
    # each token's output depends only on its own row: a subset run gives
    # bit-identical rows (the property the full-size GPU test relies on)
    xn, w1, b1, w2, b2, ids, _ = _moe_case(7, 64, 16, 24, 4)
    route = orc.hash_route(ids, 4)
    out, pre, _ = orc.moe_fwd(xn, w1, b1, w2, b2, route, 24)
    sub = np.array([3, 10, 11, 40, 63])
    out_s, pre_s, _ = orc.moe_fwd(np.ascontiguousarray(xn[sub]), w1, b1, w2, b2,
                                  np.ascontiguousarray(route[sub]), 24)
    np.testing.assert_array_equal(out_s, out[sub])
    np.testing.assert_array_equal(pre_s, pre[sub])


def test_buckets_match_reference_construction(orc):
    ids = np.random.default_rng(3).integers(0, 256, 500).astype(np.uint32)
    for E in (1, 3, 16):
        route = orc.hash_route(ids, E)
        ref = [[] for _ in range(E)]
        for t in range(len(ids)):
            ref[route[t]].append(t)
        perm, off = orc.buckets(route, E)
        assert off[0] == 0 and off[-1] == len(ids)
        for e in range(E):
            assert perm[off[e]:off[e + 1]].tolist() == ref[e]


@pytest.mark.parametrize("T,V", [(1, 7), (37, 256), (64, 1000)])
def test_cross_entropy_oracle_against_torch(orc, T, V):
    rng = np.random.default_rng(T + V)
    logits = (3 * rng.standard_normal((T, V))).astype(np.float32)
    targets = rng.integers(0, V, T).astype(np.uint32)
    loss, dl = orc.cross_entropy(logits, targets)
    x = torch.tensor(logits, dtype=torch.float64, requires_grad=True)
    ref = torch.nn.functional.cross_entropy(x, torch.tensor(targets.astype(np.int64)))
    ref.backward()
    assert abs(loss - ref.item()) <= 1e-5 * max(1.0, abs(ref.item()))
    assert orc.rel_err(dl, x.grad.numpy()) <= 1e-5
