"""Chunked (WY/UT) form of the gated delta rule, forward and backward, in
float64 numpy -- TEST INFRASTRUCTURE ONLY.

The reference specifies the chunked form without implementing it
(docs/SPEC_V2.md:50-69): with gamma_t = prod_{m<=t} alpha_m inside a chunk of C
steps, Gamma[t, i] = gamma_t / gamma_i (i <= t),

    L   = strict_tril(diag(beta) (Gamma o K K^T))
    U   = (I + L)^-1 diag(beta) (V - diag(gamma) K S)
    O   = diag(gamma) Q S + tril(Gamma o Q K^T) U
    S'  = gamma_C S + Ktilde^T U,   Ktilde = diag(Gamma[C, :]) K.

This module restates it in the phase order the GPU path uses, so every device
intermediate has a float64 counterpart:

  per chunk (independent): T = (I + L)^-1, M = tril(Gamma o Q K^T),
      Uv = T diag(beta) V, W = T diag(beta gamma) K, Qp = diag(gamma) Q - M W,
      G = Ktilde^T W, H = Ktilde^T Uv
  per unit, over chunks:   S_{c+1} = (gamma_C I - G_c) S_c + H_c
  per chunk:               O = Qp S_c + M Uv
and backward
  per chunk:               E_c = Qp^T dO_c
  per unit, reversed:      dS_c = E_c + (gamma_C I - G_c)^T dS_{c+1}
  per chunk:               the gradients of q, k, v, alpha, beta (see bwd()).

It is pinned in tests/test_oracle_chunked.py against the recurrent oracle
(oracle.c, the reference's DeltaBlock::scan_cpu / bptt_cpu restatement) and
against float64 torch autograd of the recurrence.
"""
from __future__ import annotations

import numpy as np


def _chunk_consts(alpha, beta):
    """gamma (C,), Gamma (C, C) lower incl. diagonal, via running products."""
    C = alpha.shape[0]
    gamma = np.cumprod(alpha)
    Gam = np.zeros((C, C))
    for i in range(C):
        Gam[i, i] = 1.0
        for t in range(i + 1, C):
            Gam[t, i] = Gam[t - 1, i] * alpha[t]
    return gamma, Gam


def chunk_fwd_parts(q, k, v, alpha, beta):
    """State-independent parts of one chunk (q, k, v: (C, d); alpha, beta: (C,))."""
    C = q.shape[0]
    gamma, Gam = _chunk_consts(alpha, beta)
    A = k @ k.T
    L = np.tril(beta[:, None] * Gam * A, -1)
    T = np.linalg.inv(np.eye(C) + L)
    M = np.tril(Gam * (q @ k.T))
    Uv = T @ (beta[:, None] * v)
    W = T @ ((beta * gamma)[:, None] * k)
    Qp = gamma[:, None] * q - M @ W
    gt = Gam[C - 1, :]
    Kt = gt[:, None] * k
    G = Kt.T @ W
    H = Kt.T @ Uv
    return dict(gamma=gamma, Gam=Gam, A=A, L=L, T=T, M=M, Uv=Uv, W=W, Qp=Qp, gt=gt, Kt=Kt, G=G, H=H,
                gC=gamma[C - 1])


def split(x, B, T, H, dh):
    """(B*T, H*dh) -> (B, H, T, dh)."""
    return x.reshape(B, T, H, dh).transpose(0, 2, 1, 3)


def merge(x):
    B, H, T, dh = x.shape
    return x.transpose(0, 2, 1, 3).reshape(B * T, H * dh)


def fwd(q, k, v, alpha, beta, B, T, H, dh, C):
    """Forward of all units; returns (o, cache).  alpha/beta: (B*T, H)."""
    q, k, v = (split(np.asarray(x, np.float64), B, T, H, dh) for x in (q, k, v))
    al = np.asarray(alpha, np.float64).reshape(B, T, H).transpose(0, 2, 1)
    be = np.asarray(beta, np.float64).reshape(B, T, H).transpose(0, 2, 1)
    o = np.zeros_like(q)
    cache = {}
    for b in range(B):
        for h in range(H):
            S = np.zeros((dh, dh))
            for c0 in range(0, T, C):
                sl = slice(c0, min(T, c0 + C))
                P = chunk_fwd_parts(q[b, h, sl], k[b, h, sl], v[b, h, sl], al[b, h, sl], be[b, h, sl])
                o[b, h, sl] = P["Qp"] @ S + P["M"] @ P["Uv"]
                P["S"] = S
                cache[(b, h, c0)] = P
                S = (P["gC"] * np.eye(dh) - P["G"]) @ S + P["H"]
            cache[(b, h, "final")] = S
    return merge(o), dict(parts=cache, q=q, k=k, v=v, al=al, be=be, B=B, T=T, H=H, dh=dh, C=C)


def bwd(cache, d_o):
    """Raw gradients (dq, dk, dv, dalpha, dbeta) given dO, no gradient on the
    final state (the reference's BPTT starts from dS = 0)."""
    B, T, H, dh, C = (cache[x] for x in ("B", "T", "H", "dh", "C"))
    q, k, v, al, be = (cache[x] for x in ("q", "k", "v", "al", "be"))
    dO = split(np.asarray(d_o, np.float64), B, T, H, dh)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(q), np.zeros_like(q)
    da, db = np.zeros_like(al), np.zeros_like(al)
    for b in range(B):
        for h in range(H):
            starts = list(range(0, T, C))
            dSn = np.zeros((dh, dh))  # gradient of the state after the current chunk
            for c0 in reversed(starts):
                sl = slice(c0, min(T, c0 + C))
                P = cache["parts"][(b, h, c0)]
                g = chunk_bwd(P, q[b, h, sl], k[b, h, sl], v[b, h, sl], al[b, h, sl], be[b, h, sl],
                              dO[b, h, sl], dSn)
                dq[b, h, sl], dk[b, h, sl], dv[b, h, sl], da[b, h, sl], db[b, h, sl] = g[:5]
                dSn = g[5]
    tr = lambda x: x.transpose(0, 2, 1).reshape(B * T, H)
    return merge(dq), merge(dk), merge(dv), tr(da), tr(db)


def chunk_bwd(P, q, k, v, alpha, beta, dO, dSn):
    """Gradients of one chunk given dO and dS' (state after the chunk); also
    returns dS (state before the chunk)."""
    C = q.shape[0]
    S, T_, M, Uv, W, Gam, gamma, gt, Kt, gC = (P[x] for x in ("S", "T", "M", "Uv", "W", "Gam", "gamma", "gt",
                                                               "Kt", "gC"))
    dS = P["Qp"].T @ dO + (gC * np.eye(S.shape[0]) - P["G"]).T @ dSn
    U = Uv - W @ S
    dU = M.T @ dO + Kt @ dSn
    dM = np.tril(dO @ U.T)
    dW = -dU @ S.T
    Y = T_.T @ dU
    Z = T_.T @ dW
    dv = beta[:, None] * Y
    dKt = U @ dSn.T
    Pqs = q @ S
    GdM = Gam * dM
    dq = gamma[:, None] * (dO @ S.T) + GdM @ k
    dL = np.tril(-(Y @ Uv.T + Z @ W.T), -1)
    A = P["A"]
    dA = dL * beta[:, None] * Gam
    dk = (beta * gamma)[:, None] * Z + GdM.T @ q + (dA + dA.T) @ k + gt[:, None] * dKt
    dbeta = np.sum(Y * v, 1) + gamma * np.sum(Z * k, 1) + np.sum(dL * Gam * A, 1)
    dgamma = beta * np.sum(Z * k, 1) + np.sum(dO * Pqs, 1)
    dgamma[C - 1] += np.sum(dSn * S)
    dGam = dM * (q @ k.T) + dL * beta[:, None] * A
    dGam[C - 1, :] += np.sum(k * dKt, 1)
    # dalpha_m: the derivative of every running product with alpha_m left out,
    #   d gamma_t / d alpha_m = gamma_{m-1} Gam[t, m]             (t >= m)
    #   d Gam[t, i] / d alpha_m = Gam[m-1, i] Gam[t, m]          (i < m <= t)
    # (no division by alpha: exact at alpha_m = 0)
    dGs = np.tril(dGam, -1)
    gprev = np.concatenate([[1.0], gamma[:-1]])
    dalpha = np.zeros(C)
    for m in range(C):
        r_m = np.sum(Gam[m:, m] * (dGs[m:, :m] @ Gam[m - 1, :m])) if m else 0.0
        dalpha[m] = gprev[m] * np.sum(Gam[m:, m] * dgamma[m:]) + r_m
    return dq, dk, dv, dalpha, dbeta, dS
