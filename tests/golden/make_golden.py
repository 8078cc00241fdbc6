"""Writes the golden fixtures under tests/golden/ from implementations that
share no code with the C oracle:

  * rng.json       -- Rng::next_u64 streams (rust/src/tensor.rs:307-320) for
                      seeds 0..3 in exact Python integer arithmetic, and
                      Rng::normal values (:328-332) evaluated in float64 from
                      the same integer stream;
  * hash.json      -- hash_route (rust/src/model.rs:69-77) for ids 0..4095 and
                      n_experts in {2, 8, 16}, in Python integers;
  * delta_tiny.npz -- a small gated delta-rule problem (B=2, T=12, H=2, dh=8)
                      whose forward is the matrix form of rust/src/delta.rs:1-14
                      evaluated in float64 with torch, and whose gradients come
                      from torch autograd (not from a hand derivation): raw
                      per-head gradients, and gradients through the per-head L2
                      normalisation (delta.rs:145-165) and the sigmoid gates
                      (delta.rs:167-179) for the fused variant;
  * decode_tiny.npz -- the one-token state update of DeltaBlock::step
                      (delta.rs:356-407) applied token by token in float64.

Run: python tests/golden/make_golden.py   (CPU only, a few seconds)
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent
M64 = (1 << 64) - 1


class PyRng:
    """xorshift128+ exactly as rust/src/tensor.rs:307-320, in Python ints."""

    def __init__(self, seed: int):
        self.s0 = ((seed * 0x9E3779B97F4A7C15) & M64) | 1
        self.s1 = (((seed ^ 0xDEADBEEFCAFEF00D) * 0xBF58476D1CE4E5B9) & M64) | 1

    def next_u64(self) -> int:
        x, y = self.s0, self.s1
        self.s0 = y
        x ^= (x << 23) & M64
        self.s1 = x ^ y ^ (x >> 17) ^ (y >> 26)
        return (self.s1 + y) & M64

    def uniform(self) -> float:
        return (self.next_u64() >> 40) / float(1 << 24)

    def normal64(self) -> float:
        u1 = max(self.uniform(), float(np.float32(1e-7)))
        u2 = self.uniform()
        return math.sqrt(-2.0 * math.log(u1)) * math.cos(2.0 * math.pi * u2)


def hash_route(i: int, n: int) -> int:
    h = (i * 0x9E3779B1) & 0xFFFFFFFF
    h ^= h >> 15
    h = (h * 0x85EBCA6B) & 0xFFFFFFFF
    h ^= h >> 13
    return h % n


def normals32(rng: PyRng, n: int) -> np.ndarray:
    return np.array([rng.normal64() for _ in range(n)], dtype=np.float64).astype(np.float32)


def delta_forward_torch(q, k, v, alpha, beta):
    """o (B,T,H,dh) for q,k,v (B,T,H,dh) and gates (B,T,H), S_0 = 0."""
    import torch

    B, T, H, dh = q.shape
    S = torch.zeros(B, H, dh, dh, dtype=q.dtype)
    outs = []
    for t in range(T):
        kt, vt, qt = k[:, t], v[:, t], q[:, t]
        at, bt = alpha[:, t][..., None], beta[:, t][..., None]
        sk = torch.einsum("bhai,bha->bhi", S, kt)
        u = bt * (vt - at * sk)
        S = at[..., None] * S + kt[..., :, None] * u[..., None, :]
        outs.append(torch.einsum("bhai,bha->bhi", S, qt))
    return torch.stack(outs, dim=1), S


def make_delta_tiny():
    import torch

    B, T, H, dh = 2, 12, 2, 8
    rng = PyRng(7)
    rows, d = B * T, H * dh
    q_raw = normals32(rng, rows * d).reshape(rows, d)
    k_raw = normals32(rng, rows * d).reshape(rows, d)
    v = normals32(rng, rows * d).reshape(rows, d)
    ga = (normals32(rng, rows * H) + np.float32(2.0)).reshape(rows, H)
    gb = normals32(rng, rows * H).reshape(rows, H)
    d_o = normals32(rng, rows * d).reshape(rows, d)

    # float32 normalisation / sigmoid as the forward does it, for the raw-gradient set
    def l2n32(x):
        x4 = x.reshape(rows, H, dh).astype(np.float32)
        n = np.maximum(np.sqrt((x4.astype(np.float64) ** 2).sum(-1)), 1e-8).astype(np.float32)
        return (x4 / n[..., None]).reshape(rows, d).astype(np.float32), n

    qn32, qnorm = l2n32(q_raw)
    kn32, knorm = l2n32(k_raw)
    a32 = (1.0 / (1.0 + np.exp(-ga.astype(np.float64)))).astype(np.float32)
    b32 = (1.0 / (1.0 + np.exp(-gb.astype(np.float64)))).astype(np.float32)

    def to4(x, w):
        return torch.tensor(x.astype(np.float64)).reshape(B, T, H, w) if w else torch.tensor(
            x.astype(np.float64)).reshape(B, T, H)

    # raw gradients of L = sum(o * dO) w.r.t. normalised q, k, v and alpha, beta
    qt = to4(qn32, dh).requires_grad_(True)
    kt = to4(kn32, dh).requires_grad_(True)
    vt = to4(v, dh).requires_grad_(True)
    at = to4(a32, 0).requires_grad_(True)
    bt = to4(b32, 0).requires_grad_(True)
    o, s_final = delta_forward_torch(qt, kt, vt, at, bt)
    (o * to4(d_o, dh)).sum().backward()
    raw = {
        "o": o.detach().reshape(rows, d).numpy(),
        "dq": qt.grad.reshape(rows, d).numpy(),
        "dk": kt.grad.reshape(rows, d).numpy(),
        "dv": vt.grad.reshape(rows, d).numpy(),
        "dalpha": at.grad.reshape(rows, H).numpy(),
        "dbeta": bt.grad.reshape(rows, H).numpy(),
        "s_final": s_final.detach().numpy(),
    }

    # fused gradients: w.r.t. raw q, k (through L2 norm) and gate logits (through sigmoid)
    qr = to4(q_raw, dh).requires_grad_(True)
    kr = to4(k_raw, dh).requires_grad_(True)
    vr = to4(v, dh).requires_grad_(True)
    gar = to4(ga, 0).requires_grad_(True)
    gbr = to4(gb, 0).requires_grad_(True)
    qh = qr / torch.clamp(qr.norm(dim=-1, keepdim=True), min=1e-8)
    kh = kr / torch.clamp(kr.norm(dim=-1, keepdim=True), min=1e-8)
    o2, _ = delta_forward_torch(qh, kh, vr, torch.sigmoid(gar), torch.sigmoid(gbr))
    (o2 * to4(d_o, dh)).sum().backward()
    d_qkv = np.concatenate([qr.grad.reshape(rows, d).numpy(), kr.grad.reshape(rows, d).numpy(),
                            vr.grad.reshape(rows, d).numpy()], axis=1)
    d_gate = np.concatenate([gar.grad.reshape(rows, H).numpy(), gbr.grad.reshape(rows, H).numpy()], axis=1)

    np.savez(OUT / "delta_tiny.npz", B=B, T=T, H=H, dh=dh,
             q_raw=q_raw, k_raw=k_raw, v=v, gate_a=ga, gate_b=gb, d_o=d_o,
             q=qn32, k=kn32, qnorm=qnorm, knorm=knorm, alpha=a32, beta=b32,
             d_qkv=d_qkv, d_gate=d_gate, **raw)


def make_decode_tiny():
    """Token-by-token state update of DeltaBlock::step from raw qkv rows and
    gate logits, float64, for n_seq=3, H=2, dh=8, 10 steps."""
    n_seq, H, dh, steps = 3, 2, 8, 10
    d = H * dh
    rng = PyRng(11)
    qkv = normals32(rng, steps * n_seq * 3 * d).reshape(steps, n_seq, 3 * d)
    gate = normals32(rng, steps * n_seq * 2 * H).reshape(steps, n_seq, 2 * H)
    gate[..., :H] += np.float32(2.0)
    S = np.zeros((n_seq, H, dh, dh))
    outs = []
    for s in range(steps):
        o = np.zeros((n_seq, d))
        for n in range(n_seq):
            row = qkv[s, n].astype(np.float64)
            g = gate[s, n].astype(np.float64)
            for h in range(H):
                a = 1.0 / (1.0 + math.exp(-g[h]))
                b = 1.0 / (1.0 + math.exp(-g[H + h]))
                qv = row[h * dh:(h + 1) * dh]
                kv = row[d + h * dh:d + (h + 1) * dh]
                vv = row[2 * d + h * dh:2 * d + (h + 1) * dh]
                qv = qv / max(np.linalg.norm(qv), 1e-8)
                kv = kv / max(np.linalg.norm(kv), 1e-8)
                sk = S[n, h].T @ kv
                u = b * (vv - a * sk)
                S[n, h] = a * S[n, h] + np.outer(kv, u)
                o[n, h * dh:(h + 1) * dh] = S[n, h].T @ qv
        outs.append(o)
    np.savez(OUT / "decode_tiny.npz", n_seq=n_seq, H=H, dh=dh, qkv=qkv, gate=gate,
             o=np.stack(outs), s_final=S)


def main():
    rngs = {}
    for seed in range(4):
        r = PyRng(seed)
        rngs[str(seed)] = [str(r.next_u64()) for _ in range(8)]
    normals = {}
    for seed in (0, 1):
        r = PyRng(seed)
        normals[str(seed)] = [r.normal64() for _ in range(16)]
    (OUT / "rng.json").write_text(json.dumps({"u64": rngs, "normal_f64": normals}, indent=1))
    hashes = {str(n): [hash_route(i, n) for i in range(4096)] for n in (2, 8, 16)}
    (OUT / "hash.json").write_text(json.dumps(hashes))
    make_delta_tiny()
    make_decode_tiny()
    print("golden fixtures written to", OUT)


if __name__ == "__main__":
    main()
