"""CPU restatement of the ASCA model's training step -- TEST INFRASTRUCTURE ONLY.

Composes the C oracle (oracle.c via pyoracle) into Model::forward /
Model::backward / the AdamW step of the reference (rust/src/model.rs:528-802,
rust/src/delta.rs:121-207,615-674, rust/src/train.rs:176-186).  The dense
products Mat::matmul / matmul_ta / matmul_t (rust/src/tensor.rs:91-201) are
numpy float32 matrix products here -- the same contraction, summed in a
different order, which stays orders of magnitude inside the parity bars.
Bias gradients are column sums (delta.rs:623-628,655-666).

Pinned by tests/test_oracle_model.py: a restatement of the reference's own
finite-difference model check (rust/tests/gradcheck_model.rs) and the
per-tensor AdamW step counter.  Only tests/ and bench.py's cpu_baseline leg
use this module.
"""
from __future__ import annotations

import numpy as np

from . import pyoracle as orc

_f = np.float32
EPS = 1e-6  # model.rs:14


def tensor_names(n_layers: int) -> list[str]:
    names = ["embed", "head"]
    for _ in range(n_layers):
        names += ["delta.w_qkv", "delta.b_qkv", "delta.w_gate", "delta.b_gate", "delta.w_o", "delta.b_o",
                  "moe.w1", "moe.b1", "moe.w2", "moe.b2"]
    return names


def tensor_shapes(V, d, H, L, E, dff) -> list[tuple[int, int]]:
    shp = [(V, d), (d, V)]
    for _ in range(L):
        shp += [(d, 3 * d), (1, 3 * d), (d, 2 * H), (1, 2 * H), (d, d), (1, d), (d, E * dff), (1, E * dff),
                (E * dff, d), (1, d)]
    return shp


def init_params(seed: int, V, d, H, L, E, dff) -> list[np.ndarray]:
    """Model::new's initialisation (model.rs:560-590, delta.rs:66-94,
    model.rs:88-101) drawn from the restated Rng in the same order."""
    shapes = tensor_shapes(V, d, H, L, E, dff)
    total = sum(r * c for r, c in shapes)
    z = orc.rng_normal(seed, total)  # one normal stream, consumed in order
    pos = 0

    def take(n, scale):
        nonlocal pos
        out = (z[pos:pos + n] * _f(scale)).astype(_f)
        pos += n
        return out

    out = []
    out.append(take(V * d, 0.02).reshape(V, d))
    out.append(take(d * V, np.sqrt(_f(1.0) / _f(d))).reshape(d, V))
    for _ in range(L):
        s = np.sqrt(_f(1.0) / _f(d))
        w_qkv = take(d * 3 * d, s).reshape(d, 3 * d)
        w_gate = take(d * 2 * H, s).reshape(d, 2 * H)
        w_o = take(d * d, s).reshape(d, d)
        b_gate = np.concatenate([np.full(H, -2.0, _f), np.full(H, -1.0, _f)]).reshape(1, 2 * H)
        w1 = take(d * E * dff, s).reshape(d, E * dff)
        w2 = take(E * dff * d, np.sqrt(_f(1.0) / _f(dff))).reshape(E * dff, d)
        out += [w_qkv, np.zeros((1, 3 * d), _f), w_gate, b_gate, w_o, np.zeros((1, d), _f), w1,
                np.zeros((1, E * dff), _f), w2, np.zeros((1, d), _f)]
    return out


def _sigmoid(x):
    return (_f(1.0) / (_f(1.0) + np.exp(-x))).astype(_f)


class OracleModel:
    def __init__(self, V, d, H, L, E, dff, params):
        self.V, self.d, self.H, self.L, self.E, self.dff = V, d, H, L, E, dff
        self.dh = d // H
        self.p = [np.ascontiguousarray(a, dtype=_f) for a in params]

    def _layer(self, l):
        return self.p[2 + 10 * l: 12 + 10 * l]

    def forward(self, ids, batch):
        V, d, H, dh, E, dff = self.V, self.d, self.H, self.dh, self.E, self.dff
        T = len(ids)
        seq = T // batch
        ids = np.asarray(ids, dtype=np.uint32)
        x = np.ascontiguousarray(self.p[0][ids])
        route = orc.hash_route(ids, E)
        caches = []
        for l in range(self.L):
            w_qkv, b_qkv, w_gate, b_gate, w_o, b_o, w1, b1, w2, b2 = self._layer(l)
            qkv = (x @ w_qkv + b_qkv).astype(_f)
            q, qn = orc.l2norm_heads(np.ascontiguousarray(qkv[:, :d]), H, dh)
            k, kn = orc.l2norm_heads(np.ascontiguousarray(qkv[:, d:2 * d]), H, dh)
            v = np.ascontiguousarray(qkv[:, 2 * d:])
            gate = (x @ w_gate + b_gate).astype(_f)
            alpha = np.ascontiguousarray(_sigmoid(gate[:, :H]))
            beta = np.ascontiguousarray(_sigmoid(gate[:, H:]))
            o, _ = orc.delta_scan(q, k, v, alpha, beta, batch, seq, H, dh, with_states=False)
            x_mid = (x + (o @ w_o + b_o)).astype(_f)
            xn = orc.rmsnorm(x_mid)
            out, pre, hid = orc.moe_fwd(xn, w1, np.ascontiguousarray(b1.reshape(-1)), w2,
                                        np.ascontiguousarray(b2.reshape(-1)), route, dff)
            x_out = (x_mid + out).astype(_f)
            caches.append(dict(x_in=x, q=q, k=k, v=v, qn=qn, kn=kn, alpha=alpha, beta=beta, o=o, x_mid=x_mid,
                               xn=xn, pre=pre, hid=hid))
            x = x_out
        h = orc.rmsnorm(x)
        logits = (h @ self.p[1]).astype(_f)
        return logits, dict(ids=ids, route=route, layers=caches, x_last=x, h=h, batch=batch, seq=seq)

    def loss(self, ids, targets, batch=1):
        logits, _ = self.forward(ids, batch)
        loss, _ = orc.cross_entropy(logits, targets)
        return loss

    def forward_backward(self, ids, targets, batch):
        """(loss, grads in params() order) after zero_grads."""
        d, H, dh, dff = self.d, self.H, self.dh, self.dff
        logits, c = self.forward(ids, batch)
        loss, dlogits = orc.cross_entropy(logits, targets)
        g = [np.zeros_like(a) for a in self.p]
        g[1] = (c["h"].T @ dlogits).astype(_f)
        dx = orc.rmsnorm_bwd(c["x_last"], (dlogits @ self.p[1].T).astype(_f))
        for l in reversed(range(self.L)):
            w_qkv, b_qkv, w_gate, b_gate, w_o, b_o, w1, b1, w2, b2 = self._layer(l)
            lc = c["layers"][l]
            dxn, dw1, db1, dw2, db2 = orc.moe_bwd(lc["xn"], w1, w2, lc["pre"], lc["hid"], c["route"], dx, dff)
            d_mid = (dx + orc.rmsnorm_bwd(lc["x_mid"], dxn)).astype(_f)
            d_o = np.ascontiguousarray((d_mid @ w_o.T).astype(_f))
            gw_o = (lc["o"].T @ d_mid).astype(_f)
            gb_o = d_mid.sum(axis=0, dtype=_f).reshape(1, -1)
            _, dq, dk, dv, da, db = orc.delta_fwd_bwd(lc["q"], lc["k"], lc["v"], lc["alpha"], lc["beta"], d_o,
                                                      c["batch"], c["seq"], H, dh)
            d_qkv, d_gate = orc.delta_fuse(lc["q"], lc["k"], lc["qn"], lc["kn"], lc["alpha"], lc["beta"], dq, dk,
                                           dv, da, db, H, dh)
            x_in = lc["x_in"]
            base = 2 + 10 * l
            g[base + 0] = (x_in.T @ d_qkv).astype(_f)
            g[base + 1] = d_qkv.sum(axis=0, dtype=_f).reshape(1, -1)
            g[base + 2] = (x_in.T @ d_gate).astype(_f)
            g[base + 3] = d_gate.sum(axis=0, dtype=_f).reshape(1, -1)
            g[base + 4] = gw_o
            g[base + 5] = gb_o
            g[base + 6] = dw1
            g[base + 7] = db1.reshape(1, -1)
            g[base + 8] = dw2
            g[base + 9] = db2.reshape(1, -1)
            dx = (d_mid + ((d_qkv @ w_qkv.T).astype(_f) + (d_gate @ w_gate.T).astype(_f))).astype(_f)
        ge = np.zeros_like(self.p[0])
        np.add.at(ge, c["ids"], dx)  # row by row in token order (model.rs:782-789)
        g[0] = ge
        return loss, g

    def adamw(self, grads, m, v, step, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.01):
        """model::step: AdamW::update on every tensor in params() order, the
        step counter advancing per tensor; returns the new counter."""
        for i in range(len(self.p)):
            p = self.p[i].reshape(-1)
            step = orc.adamw(p, np.ascontiguousarray(grads[i].reshape(-1)), m[i].reshape(-1), v[i].reshape(-1),
                             lr, step, beta1, beta2, eps, wd)
        return step
