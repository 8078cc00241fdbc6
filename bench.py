#!/usr/bin/env python3
"""Headline benchmark: gated delta-rule fwd + BPTT, f32, at B=32 T=512 H=8
dh=64 (seed 1) on one MI355X.  The recurrence runs over T
with each (sequence, head) state resident in registers, advanced 16 steps per
block on the f32 matrix cores (the UT form of the same recurrence).

A step is one forward (asca_delta_fwd) plus one BPTT with the fused L2-norm and
sigmoid backward (asca_delta_bwd_fused, the drop-in for Gpu::delta_bwd_dev) over
one batch of synthetic inputs already resident in HBM.  An untimed steady-clock
prewarm and W untimed warm-up steps, then K timed steps on one stream with nothing
else on it; then a second pass of K steps with a HIP event around each launch gives
the kernel durations (an event record between kernels costs stream time, so the
timed region has none).  Prints one JSON line.

The CPU baseline is the oracle's restatement of the reference CPU path
(DeltaBlock::scan_cpu + bptt_cpu with its thread decomposition) on the same
inputs, timed on this host in the same run.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "delta fwd+BPTT tokens/s (B32 T512 H8 dh64 f32) + % of roofline"
PEAK_F32 = 157.3e12   # MI355X published dense fp32 peak (matrix cores / packed VALU), FLOP/s
PEAK_HBM = 8.0e12     # MI355X HBM3E, B/s
HEADLINE = dict(B=32, T=512, H=8, dh=64, seed=1)
PMC_FILE = ROOT / "profiles" / "delta_b32t512h8d64_traffic.json"
# the sources of the delta kernels: counters measured on other sources are stale
KERNEL_SOURCES = ["asca_amd/csrc/delta.hip", "asca_amd/csrc/delta_ut64.hip", "asca_amd/csrc/ut64_kernels.h",
                  "asca_amd/csrc/delta_ut64_b.hip", "asca_amd/csrc/delta.h", "asca_amd/csrc/common.h",
                  "asca_amd/build.py"]


def kernel_sources_sha() -> str:
    import hashlib

    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()[:16]


def synth_inputs(B, T, H, dh, seed):
    """configs[1] inputs drawn from the reference's Rng stream (product
    restatement in libasca_hip): q, k, v ~ N(0,1); alpha logits 2+N(0,1);
    beta logits N(0,1); dO ~ N(0,1); then per-head L2 norm of q, k and
    sigmoid gates."""
    from asca_amd import _lib

    lib = _lib.load()
    st = (C.c_uint64 * 2)()
    lib.asca_rng_seed(seed, st)
    rows, d = B * T, H * dh

    def normal(n, scale=1.0, offset=0.0):
        out = np.empty(n, dtype=np.float32)
        lib.asca_rng_normal(st, out.ctypes.data_as(C.c_void_p), n, scale, offset)
        return out

    q = normal(rows * d).reshape(rows, d)
    k = normal(rows * d).reshape(rows, d)
    v = normal(rows * d).reshape(rows, d)
    ga = normal(rows * H, 1.0, 2.0).reshape(rows, H)
    gb = normal(rows * H).reshape(rows, H)
    d_o = normal(rows * d).reshape(rows, d)

    def l2n(x):
        x3 = x.reshape(rows, H, dh)
        n = np.maximum(np.sqrt(np.einsum("rhc,rhc->rh", x3, x3, dtype=np.float32)), np.float32(1e-8))
        return np.ascontiguousarray((x3 / n[..., None]).reshape(rows, d), dtype=np.float32), n.astype(np.float32)

    q, qn = l2n(q)
    k, kn = l2n(k)
    alpha = (1.0 / (1.0 + np.exp(-ga))).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-gb))).astype(np.float32)
    return dict(q=q, k=k, v=v, alpha=alpha, beta=beta, d_o=d_o, qn=qn, kn=kn)


def work_model(B, T, H, dh):
    """Algorithmic work (rust/src/delta.rs:289-314 forward, :504-564 BPTT):
    7 dh^2 + 17 dh^2 flops per token-head; compulsory bytes per token-head:
    fwd reads q,k,v (3 dh) + alpha,beta, writes o (dh); BPTT reads q,k,v,dO
    (4 dh) + alpha,beta, writes dq,dk,dv (3 dh) + dalpha,dbeta."""
    th = B * T * H
    f_fwd, f_bwd = 7 * dh * dh * th, 17 * dh * dh * th
    b_fwd = (3 * dh * 4 + 8 + dh * 4) * th
    b_bwd = (4 * dh * 4 + 8 + 3 * dh * 4 + 8) * th
    return f_fwd, f_bwd, b_fwd, b_bwd


def cpu_baseline(x, B, T, H, dh, budget_s=30.0):
    """The reference CPU path restated in C (oracle), reference threading:
    one thread per head in the scan, one per (head, sequence) in the BPTT,
    full state history kept as the reference does.  Median of >= 5 reps after
    one warm-up (fewer only if one rep exceeds the budget)."""
    from oracle import pyoracle as orc

    def once():
        t0 = time.perf_counter()
        o, st = orc.delta_scan(x["q"], x["k"], x["v"], x["alpha"], x["beta"], B, T, H, dh)
        raw = orc.delta_bptt_raw(x["q"], x["k"], x["v"], x["alpha"], x["beta"], x["d_o"], st, B, T, H, dh)
        orc.delta_fuse(x["q"], x["k"], x["qn"], x["kn"], x["alpha"], x["beta"], *raw, H, dh)
        return time.perf_counter() - t0

    once()
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - t_start) < budget_s:
        times.append(once())
    med = statistics.median(times)
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {
        "value": round(B * T / med, 1),
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"full configs[1] workload (B{B} T{T} H{H} dh{dh}, same inputs), oracle restatement of "
                   f"scan_cpu + bptt_cpu + norm/sigmoid backward with the reference's threads "
                   f"({H} scan threads, {H * B} BPTT threads) on {cores} host cores; median of {len(times)} reps "
                   f"after 1 warm-up, {med:.3f} s each; AVX2={bool(orc.lib().orc_has_avx2())}"),
    }


class Timer:
    """HIP events on one stream of the library (no torch in this process)."""

    def __init__(self):
        from asca_amd import _lib

        self._lib = _lib
        sp = C.c_void_p()
        _lib.call("asca_stream_create", C.byref(sp))
        self.stream = sp.value

    def event(self):
        e = C.c_void_p()
        self._lib.call("asca_event_create", C.byref(e))
        return e

    def record(self, e):
        self._lib.call("asca_event_record", e, C.c_void_p(self.stream))

    def elapsed(self, a, b):
        ms = C.c_float()
        self._lib.call("asca_event_elapsed_ms", C.byref(ms), a, b)
        return ms.value

    def sync(self):
        self._lib.call("asca_stream_sync", C.c_void_p(self.stream))

    def destroy(self, *evs):
        for e in evs:
            self._lib.call("asca_event_destroy", e)


def bench_decode(args):
    """batched single-token decode, 512 sequences, H=16, dh=128,
    persistent f32 states in HBM; one step reads and writes every state once.
    Inputs (q, k, v normals, alpha logits 2+N, beta logits N, seed 3) come
    from the reference Rng stream; a pool of 8 steps' inputs is cycled."""
    from asca_amd import _lib, gpu
    from asca_amd.gpu import DevBuf

    g = gpu.gpu()
    if g is None:
        raise SystemExit(f"no GPU backend: {gpu.describe()}")
    n, H, dh, seed, pool = 512, 16, 128, 3, 8
    d = H * dh
    lib = _lib.load()
    st = (C.c_uint64 * 2)()
    lib.asca_rng_seed(seed, st)
    qkvs, gates = [], []
    for _ in range(pool):
        qkv = np.empty((n, 3 * d), dtype=np.float32)
        lib.asca_rng_normal(st, qkv.ctypes.data_as(C.c_void_p), qkv.size, 1.0, 0.0)
        gate = np.empty((n, 2 * H), dtype=np.float32)
        lib.asca_rng_normal(st, gate.ctypes.data_as(C.c_void_p), gate.size, 1.0, 0.0)
        gate[:, :H] += 2.0
        qkvs.append(qkv)
        gates.append(gate)
    dq = [DevBuf.from_host(x) for x in qkvs]
    dg = [DevBuf.from_host(x) for x in gates]
    states = g.new_decode_states(n, H, dh)
    o = DevBuf(n * d * 4)
    tm = Timer()

    def step(i):
        _lib.call("asca_delta_decode_step", C.c_void_p(states.ptr), C.c_void_p(dq[i % pool].ptr),
                  C.c_void_p(dg[i % pool].ptr), C.c_void_p(o.ptr), n, H, dh, C.c_void_p(tm.stream))

    K = args.steps or 256
    W = args.warmup
    print(f"bench decode: {gpu.describe()}; n{n} H{H} dh{dh}; warmup {W}, steps {K}", flush=True)
    for i in range(W):
        step(i)
    tm.sync()
    e0, e1 = tm.event(), tm.event()
    t0 = time.perf_counter()
    tm.record(e0)
    for i in range(K):
        step(i)
    tm.record(e1)
    tm.sync()
    wall = time.perf_counter() - t0
    dev_ms = tm.elapsed(e0, e1) / K
    tm.destroy(e0, e1)
    state_bytes = 2 * n * H * dh * dh * 4
    io_bytes = n * (3 * d + 2 * H) * 4 + n * d * 4
    bytes_step = state_bytes + io_bytes
    achieved = bytes_step / (dev_ms * 1e-3)
    result = {
        "metric": "decode tokens/s (512 seq H16 dh128 f32, 256 steps) + HBM GB/s",
        "value": round(n * K / wall, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(wall / K * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (reference Rng stream, configs[4] distributions, seed 3, 8-step input pool)",
        "config": {"workload": "batched decode step (asca_delta_decode_step)", "n_seq": n, "H": H, "dh": dh},
        "roofline": {"bound": "hbm", "achieved": round(achieved / 1e9, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM, 4), "traffic": None, "kernel": "delta_decode",
                     "algorithmic_bytes": bytes_step},
        "kernels_ms": {"delta_decode": round(dev_ms, 4)},
    }
    if not args.no_cpu:
        from oracle import pyoracle as orc

        ns = 64
        S = np.zeros((ns, H, dh, dh), dtype=np.float32)
        qkv, gate = np.ascontiguousarray(qkvs[0][:ns]), np.ascontiguousarray(gates[0][:ns])
        orc.delta_decode_step(S, qkv, gate, H, dh)
        times = []
        for _ in range(5):
            t1 = time.perf_counter()
            orc.delta_decode_step(S, qkv, gate, H, dh)
            times.append(time.perf_counter() - t1)
        med = statistics.median(times)
        result["cpu_baseline"] = {
            "value": round(ns / med, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"oracle restatement of DeltaBlock::step state math, {ns} of the 512 sequences, one thread "
                      f"(the reference's decode is single-threaded per token), median of 5 steps, {med:.4f} s each"}
    print(json.dumps(result), flush=True)


def bench_chunk(args):
    """chunked (WY/UT) delta-rule fwd+BPTT, chunk 64, B=8, T=4096,
    H=16, dh=128; q, k, v, dO in bf16 (q, k L2-normalised first), gates f32;
    inputs from the reference Rng in the order of configs[0] (seed 0, the
    config states none)."""
    from asca_amd import _lib, gpu
    from asca_amd.gpu import DevBuf, to_bf16

    B, T, H, dh, Cc, seed = 8, 4096, 16, 128, 64, 0
    g = gpu.gpu()
    if g is None:
        raise SystemExit(f"no GPU backend: {gpu.describe()}")
    x = synth_inputs(B, T, H, dh, seed)
    bf = {n: to_bf16(x[n]) for n in ("q", "k", "v", "d_o")}
    dev = {n: DevBuf.from_array(a) for n, a in bf.items()}
    da, db = DevBuf.from_host(x["alpha"]), DevBuf.from_host(x["beta"])
    wsb = C.c_size_t()
    _lib.call("asca_chunk_ws_bytes", B, T, H, dh, Cc, C.byref(wsb))
    ws = DevBuf(wsb.value)
    o = DevBuf(B * T * H * dh * 4)
    grads = [DevBuf(B * T * H * dh * 4) for _ in range(3)] + [DevBuf(B * T * H * 4) for _ in range(2)]
    tm = Timer()
    sp = C.c_void_p(tm.stream)

    def fwd():
        _lib.call("asca_chunk_fwd", C.c_void_p(dev["q"].ptr), C.c_void_p(dev["k"].ptr), C.c_void_p(dev["v"].ptr),
                  C.c_void_p(da.ptr), C.c_void_p(db.ptr), C.c_void_p(o.ptr), C.c_void_p(ws.ptr), B, T, H, dh, Cc, sp)

    def bwd():
        _lib.call("asca_chunk_bwd", C.c_void_p(dev["q"].ptr), C.c_void_p(dev["k"].ptr), C.c_void_p(dev["v"].ptr),
                  C.c_void_p(dev["d_o"].ptr), C.c_void_p(ws.ptr),
                  *[C.c_void_p(b.ptr) for b in grads], B, T, H, dh, Cc, sp)

    K = args.steps or 10
    W = min(args.warmup, 3)
    print(f"bench chunk: {gpu.describe()}; B{B} T{T} H{H} dh{dh} C{Cc}; ws {wsb.value / 2**30:.2f} GiB; "
          f"warmup {W}, steps {K}", flush=True)
    for _ in range(W):
        fwd()
        bwd()
    tm.sync()
    ev = [tm.event() for _ in range(3)]
    f_ms = b_ms = 0.0
    t0 = time.perf_counter()
    for _ in range(K):
        tm.record(ev[0])
        fwd()
        tm.record(ev[1])
        bwd()
        tm.record(ev[2])
        tm.sync()
        f_ms += tm.elapsed(ev[0], ev[1])
        b_ms += tm.elapsed(ev[1], ev[2])
    wall = time.perf_counter() - t0
    tm.destroy(*ev)
    f_ms /= K
    b_ms /= K
    tokens = B * T
    flops = 24 * dh * dh * B * T * H  # 18 C d^2 + 12 C^2 d per chunk = 24 d^2 per token-head at C = d/2
    step_ms = f_ms + b_ms
    achieved = flops / (step_ms * 1e-3)
    result = {
        "metric": "chunked delta fwd+BPTT tokens/s (configs[2]: B8 T4096 H16 dh128, chunk 64, bf16 in, f32 acc)",
        "value": round(tokens * K / wall, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(wall / K * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 in / f32 MFMA",
        "data": f"synthetic (reference Rng stream, configs[0] distributions, seed {seed}), bf16-rounded",
        "config": {"workload": "chunked delta-rule fwd+BPTT (asca_chunk_fwd + asca_chunk_bwd)", "B": B, "T": T,
                   "H": H, "dh": dh, "chunk": Cc},
        "roofline": {"bound": "mfma", "achieved": round(achieved / 1e12, 2), "peak": PEAK_F32 / 1e12,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_F32, 4), "traffic": None, "kernel": "step",
                     "algorithmic_flops": flops},
        "kernels_ms": {"chunk_fwd": round(f_ms, 3), "chunk_bwd": round(b_ms, 3)},
    }
    if not args.no_cpu:
        from oracle import pyoracle as orc
        from asca_amd.gpu import from_bf16

        # the recurrent CPU path on one sequence x 4 heads of the same bf16-rounded inputs
        Hs = 4
        cols = slice(0, Hs * dh)
        sub = {n: np.ascontiguousarray(from_bf16(bf[n][:T, cols])) for n in ("q", "k", "v", "d_o")}
        a, bt = (np.ascontiguousarray(x[n][:T, :Hs]) for n in ("alpha", "beta"))
        t1 = time.perf_counter()
        orc.delta_fwd_bwd(sub["q"], sub["k"], sub["v"], a, bt, sub["d_o"], 1, T, Hs, dh, nthreads=Hs)
        el = time.perf_counter() - t1
        result["cpu_baseline"] = {
            "value": round(T * Hs / H / el, 1), "unit": "tokens/s", "cores": Hs, "kind": "port",
            "sample": f"oracle recurrent fwd+BPTT (scan_cpu + bptt_cpu restatement) on 1 sequence x {Hs} of "
                      f"the {H} heads (one thread per head), {el:.1f} s; tokens/s scaled to all {H} heads"}
    print(json.dumps(result), flush=True)


TRAIN_CFG = dict(V=256, d=512, H=8, L=8, E=16, dff=1024, B=16, T=1024, seed=2)


def train_flops_per_token(V, d, H, L, E, dff):
    """Algorithmic flops of one training step per token: every dense product
    once forward and twice backward, the recurrence's 24 dh^2 per head
    (7 forward + 17 backward, delta.rs:289-314,504-564), the output head."""
    dh = d // H
    gemm_fwd = 2 * d * 3 * d + 2 * d * 2 * H + 2 * d * d + 2 * 2 * d * dff
    return L * (3 * gemm_fwd + 24 * dh * dh * H) + 3 * 2 * d * V


def chunk_flops(B, T, H, dh, Cc):
    """MFMA flops the batched chunked path executes (its GEMM list in
    chunk.hip, forward then backward): per chunk 30 C^2 d + 20 C d^2 + 4 d^3
    (the two state scans are d x d products per chunk)."""
    nc = -(-T // Cc)
    per_chunk = 30 * Cc * Cc * dh + 20 * Cc * dh * dh + 4 * dh ** 3
    return B * H * nc * per_chunk


def bench_chunk64(args):
    """The MFMA route at the headline shape: configs[1] (B32 T512 H8 dh64, f32,
    seed 1) through the f32 chunked path (asca_chunk_fwd_f32 +
    asca_chunk_bwd_f32, batched MFMA GEMMs over chunks) at C = 16, 32, 64,
    timed next to the recurrent kernels on the same device inputs
    (asca_delta_fwd + asca_delta_bwd_raw: the same raw gradients)."""
    from asca_amd import _lib, gpu
    from asca_amd.gpu import DevBuf

    B, T, H, dh, seed = 32, 512, 8, 64, 1
    g = gpu.gpu()
    if g is None:
        raise SystemExit(f"no GPU backend: {gpu.describe()}")
    x = synth_inputs(B, T, H, dh, seed)
    dev = {n: DevBuf.from_host(x[n]) for n in ("q", "k", "v", "alpha", "beta", "d_o")}
    rows, d = B * T, H * dh
    o = DevBuf(rows * d * 4)
    grads = [DevBuf(rows * d * 4) for _ in range(3)] + [DevBuf(rows * H * 4) for _ in range(2)]
    tm = Timer()
    sp = C.c_void_p(tm.stream)
    P = {n: C.c_void_p(b.ptr) for n, b in dev.items()}
    G = [C.c_void_p(b.ptr) for b in grads]
    K = args.steps or 20
    W = min(args.warmup, 3)

    def timed(fwd, bwd):
        for _ in range(W):
            fwd()
            bwd()
        tm.sync()
        ev = [tm.event() for _ in range(3)]
        f_ms = b_ms = 0.0
        for _ in range(K):
            tm.record(ev[0])
            fwd()
            tm.record(ev[1])
            bwd()
            tm.record(ev[2])
            tm.sync()
            f_ms += tm.elapsed(ev[0], ev[1])
            b_ms += tm.elapsed(ev[1], ev[2])
        tm.destroy(*ev)
        return f_ms / K, b_ms / K

    print(f"bench chunk64: {gpu.describe()}; B{B} T{T} H{H} dh{dh} f32; warmup {W}, steps {K}", flush=True)
    per_c = {}
    for Cc in (16, 32, 64):
        wsb = C.c_size_t()
        _lib.call("asca_chunk_ws_bytes_f32", B, T, H, dh, Cc, C.byref(wsb))
        ws = DevBuf(wsb.value)
        wp = C.c_void_p(ws.ptr)

        def fwd():
            _lib.call("asca_chunk_fwd_f32", P["q"], P["k"], P["v"], P["alpha"], P["beta"], C.c_void_p(o.ptr), wp,
                      B, T, H, dh, Cc, sp)

        def bwd():
            _lib.call("asca_chunk_bwd_f32", P["d_o"], wp, *G, B, T, H, dh, Cc, sp)

        f_ms, b_ms = timed(fwd, bwd)
        ws.free()
        fl = chunk_flops(B, T, H, dh, Cc)
        per_c[Cc] = {"fwd_ms": round(f_ms, 4), "bwd_ms": round(b_ms, 4), "step_ms": round(f_ms + b_ms, 4),
                     "ws_mib": round(wsb.value / 2**20, 1), "mfma_gflop": round(fl / 1e9, 2),
                     "mfma_tflops": round(fl / ((f_ms + b_ms) * 1e-3) / 1e12, 2)}
        print(f"bench chunk64: C={Cc}: fwd {f_ms:.4f} ms, bwd {b_ms:.4f} ms, "
              f"{per_c[Cc]['mfma_tflops']} TFLOP/s MFMA", flush=True)
    # the recurrent kernels on the same inputs (raw gradients, like the chunked path)
    wsb = C.c_size_t()
    _lib.call("asca_delta_ws_bytes", B, T, H, dh, C.byref(wsb))
    ws = DevBuf(wsb.value)
    wp = C.c_void_p(ws.ptr)

    def rfwd():
        _lib.call("asca_delta_fwd", P["q"], P["k"], P["v"], P["alpha"], P["beta"], C.c_void_p(o.ptr), wp,
                  B, T, H, dh, sp)

    def rbwd():
        _lib.call("asca_delta_bwd_raw", P["q"], P["k"], P["v"], P["alpha"], P["beta"], P["d_o"], wp, *G,
                  B, T, H, dh, sp)

    rf, rb = timed(rfwd, rbwd)
    ws.free()
    print(f"bench chunk64: recurrent: fwd {rf:.4f} ms, bwd {rb:.4f} ms", flush=True)
    best = min(per_c, key=lambda c: per_c[c]["step_ms"])
    step_ms = per_c[best]["step_ms"]
    fl = chunk_flops(B, T, H, dh, best)
    result = {
        "metric": "chunked (MFMA) delta fwd+BPTT tokens/s at the headline shape (B32 T512 H8 dh64 f32)",
        "value": round(B * T / (step_ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": step_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": f"synthetic (reference Rng stream, configs[1] distributions, seed {seed})",
        "config": {"workload": "chunked delta-rule fwd+BPTT on f32 (asca_chunk_fwd_f32 + asca_chunk_bwd_f32)",
                   "B": B, "T": T, "H": H, "dh": dh, "chunk": best},
        "roofline": {"bound": "mfma", "achieved": per_c[best]["mfma_tflops"], "peak": PEAK_F32 / 1e12,
                     "unit": "TFLOP/s", "frac": round(fl / (step_ms * 1e-3) / PEAK_F32, 4), "traffic": None,
                     "kernel": "step", "algorithmic_flops": fl,
                     "note": "flops the batched chunked path executes (30 C^2 d + 20 C d^2 + 4 d^3 per chunk)"},
        "per_chunk_size": per_c,
        "recurrent_same_inputs_ms": {"delta_fwd": round(rf, 4), "delta_bwd_raw": round(rb, 4),
                                     "step": round(rf + rb, 4)},
    }
    print(json.dumps(result), flush=True)


def bench_train(args):
    """one full training step (forward, BPTT backward, AdamW over
    all 143.1M parameters) of the 8-layer model, B=16 x T=1024 byte tokens,
    weights N(0, 0.02) from the reference Rng (seed 2), targets = ids shifted
    by one (Data::batch, rust/src/train.rs:145-155)."""
    from asca_amd import _lib, gpu
    from asca_amd.gpu import DevBuf
    from asca_amd.model import DeviceModel

    c = TRAIN_CFG
    V, d, H, L, E, dff, B, T = c["V"], c["d"], c["H"], c["L"], c["E"], c["dff"], c["B"], c["T"]
    if gpu.gpu() is None:
        raise SystemExit(f"no GPU backend: {gpu.describe()}")
    lib = _lib.load()
    st = (C.c_uint64 * 2)()
    lib.asca_rng_seed(c["seed"], st)
    dm = DeviceModel(V, d, H, L, E, dff)
    params = []
    for _, _, r, cc in dm.tensors:
        a = np.empty(r * cc, dtype=np.float32)
        lib.asca_rng_normal(st, a.ctypes.data_as(C.c_void_p), a.size, 0.02, 0.0)
        params.append(a)
    dm.set_params(params)
    dm.set_adamw(3e-4)
    raw = np.empty(B * (T + 1), dtype=np.uint64)
    lib.asca_rng_u64(st, raw.ctypes.data_as(C.POINTER(C.c_uint64)), raw.size)
    toks = (raw % 256).astype(np.uint32).reshape(B, T + 1)
    ids, tgts = toks[:, :T].reshape(-1), toks[:, 1:].reshape(-1)
    di, dt = DevBuf.from_array(ids), DevBuf.from_array(tgts)
    tm = Timer()
    K = args.steps or 10
    W = args.warmup
    print(f"bench train: {gpu.describe()}; V{V} d{d} L{L} H{H} E{E} dff{dff} B{B} T{T}; "
          f"{dm.num_params()} params; warmup {W}, steps {K}", flush=True)
    for _ in range(W):
        dm.train_step_dev(di, dt, B, T, sync=False, stream=C.c_void_p(tm.stream))
    tm.sync()
    loss0 = dm._read_loss()
    e0, e1 = tm.event(), tm.event()
    t0 = time.perf_counter()
    tm.record(e0)
    for _ in range(K):
        dm.train_step_dev(di, dt, B, T, sync=False, stream=C.c_void_p(tm.stream))
    tm.record(e1)
    tm.sync()
    wall = time.perf_counter() - t0
    dev_ms = tm.elapsed(e0, e1) / K
    tm.destroy(e0, e1)
    loss = dm._read_loss()
    fpt = train_flops_per_token(V, d, H, L, E, dff)
    achieved = fpt * B * T / (dev_ms * 1e-3)
    result = {
        "metric": "training tokens/s (configs[3]: V256 d512 L8 H8 E16 dff1024, B16 T1024, f32, fwd+BPTT+AdamW)",
        "value": round(B * T * K / wall, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(wall / K * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": f"synthetic bytes from the reference Rng (seed {c['seed']}), N(0,0.02) weights; "
                f"loss {loss0:.4f} -> {loss:.4f} over the timed steps",
        "config": {"workload": "full training step (asca_model_train_step)", "global_batch": B, "seq_len": T,
                   "d_model": d, "layers": L, "heads": H, "experts": E, "d_ff": dff, "vocab": V},
        "roofline": {"bound": "mfma", "achieved": round(achieved / 1e12, 2), "peak": PEAK_F32 / 1e12,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_F32, 4), "traffic": None, "kernel": "step",
                     "algorithmic_flops_per_token": fpt},
    }
    if not args.no_cpu:
        from oracle import model_oracle as mo

        om = mo.OracleModel(V, d, H, L, E, dff, [p.reshape(r, cc) for p, (_, _, r, cc) in zip(params, dm.tensors)])
        t1 = time.perf_counter()
        om.forward_backward(ids[:T], tgts[:T], 1)
        el = time.perf_counter() - t1
        result["cpu_baseline"] = {
            "value": round(T / el, 1), "unit": "tokens/s", "cores": min(os.cpu_count() or 1, 16), "kind": "port",
            "sample": f"oracle restatement of Model::forward+backward (C oracle: delta scan/BPTT threaded per head / "
                      f"(head, seq), MoE threaded per expert; numpy f32 GEMMs), 1 of the {B} sequences "
                      f"({T} tokens), no optimiser step, {el:.1f} s"}
    dm.close()
    print(json.dumps(result), flush=True)


GEMM_SHAPES = [  # (name, trans_a, trans_b, M, N, K): the f32 products of configs[3] and a square one
    ("qkv projection 16384x1536x512 NN", 0, 0, 16384, 1536, 512),
    ("out projection 16384x512x512 NN", 0, 0, 16384, 512, 512),
    ("qkv input gradient 16384x512x1536 NT", 0, 1, 16384, 512, 1536),
    ("qkv weight gradient 512x1536x16384 TN (split-K)", 1, 0, 512, 1536, 16384),
    ("head 16384x256x512 NN", 0, 0, 16384, 256, 512),
    ("square 4096x4096x4096 NN", 0, 0, 4096, 4096, 4096),
]


def bench_gemm(args):
    """The f32 MFMA GEMM (asca_gemm) on the configs[3] product shapes and
    4096^3, operands resident in HBM, HIP events around K launches each;
    value = TFLOP/s of the 4096^3 product (the MFMA-bound reference point)."""
    from asca_amd import _lib, gpu
    from asca_amd.gpu import DevBuf

    if gpu.gpu() is None:
        raise SystemExit(f"no GPU backend: {gpu.describe()}")
    K_rep = args.steps or 20
    W = args.warmup
    rng = np.random.default_rng(0)
    tm = Timer()
    out = {}
    for name, ta, tb, M, N, K in GEMM_SHAPES:
        a = DevBuf.from_host(rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
        b = DevBuf.from_host(rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32))
        c = DevBuf(M * N * 4)
        lda, ldb = (M if ta else K), (K if tb else N)
        args_c = (ta, tb, M, N, K, C.c_float(1.0), C.c_void_p(a.ptr), lda, C.c_void_p(b.ptr), ldb, C.c_float(0.0),
                  C.c_void_p(c.ptr), N, None, C.c_void_p(tm.stream))
        for _ in range(W):
            _lib.call("asca_gemm", *args_c)
        tm.sync()
        e0, e1 = tm.event(), tm.event()
        tm.record(e0)
        for _ in range(K_rep):
            _lib.call("asca_gemm", *args_c)
        tm.record(e1)
        tm.sync()
        ms = tm.elapsed(e0, e1) / K_rep
        tm.destroy(e0, e1)
        out[name] = {"us": round(ms * 1e3, 1), "tflops": round(2.0 * M * N * K / ms / 1e9, 1)}
        print(f"bench gemm: {name}: {ms * 1e3:.1f} us, {out[name]['tflops']} TFLOP/s", file=sys.stderr, flush=True)
        a.free(), b.free(), c.free()
    sq = out["square 4096x4096x4096 NN"]
    result = {
        "metric": "f32 GEMM TFLOP/s (asca_gemm, 4096^3 NN; configs[3] product shapes alongside)",
        "value": sq["tflops"], "unit": "TFLOP/s", "n_gpus": 1, "steps": K_rep, "warmup": W,
        "ms_per_step": round(sq["us"] / 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic N(0,1) operands",
        "config": {"workload": "asca_gemm (MFMA f32)", "shapes": out},
        "roofline": {"bound": "mfma", "achieved": sq["tflops"], "peak": 157.3, "unit": "TFLOP/s",
                     "frac": round(sq["tflops"] / 157.3, 4), "traffic": None, "kernel": "gemm_k 4096^3"},
    }
    print(json.dumps(result), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="delta", choices=["delta", "decode", "train", "chunk", "chunk64", "gemm"],
                    help="delta: the headline fwd+BPTT (configs[1]); decode: configs[4]; train: configs[3]; "
                         "chunk: configs[2]; chunk64: the chunked (MFMA) form at the configs[1] shape, f32; "
                         "gemm: the f32 GEMM on the configs[3] product shapes")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--prewarm-ms", type=float, default=300.0,
                    help="untimed fwd + bwd for this long (wall ms) before the warm-up steps, to reach steady clocks")
    ap.add_argument("--calib", action="store_true",
                    help="also run the known-size copy kernel (for counter calibration)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        sys.stderr.write("bench.py: this build runs on exactly one GPU (the delta-rule units are independent "
                         "per (sequence, head), so the path would shard over B or H with no exchange). "
                         "Use --gpus 1.\n")
        sys.exit(2)
    if args.workload == "decode":
        bench_decode(args)
        return
    if args.workload == "train":
        bench_train(args)
        return
    if args.workload == "chunk64":
        bench_chunk64(args)
        return
    if args.workload == "chunk":
        bench_chunk(args)
        return
    if args.workload == "gemm":
        bench_gemm(args)
        return
    if args.steps is None:
        args.steps = 100

    from asca_amd import _lib, gpu
    from asca_amd.gpu import DevBuf

    g = gpu.gpu()
    if g is None:
        raise SystemExit(f"no GPU backend: {gpu.describe()}")
    B, T, H, dh, seed = (HEADLINE[k] for k in ("B", "T", "H", "dh", "seed"))
    rows, d = B * T, H * dh
    x = synth_inputs(B, T, H, dh, seed)
    dev = {k: DevBuf.from_host(v) for k, v in x.items()}
    wsb = C.c_size_t()
    _lib.call("asca_delta_ws_bytes", B, T, H, dh, C.byref(wsb))
    ws = DevBuf(wsb.value)
    o = DevBuf(rows * d * 4)
    d_qkv = DevBuf(rows * 3 * d * 4)
    d_gate = DevBuf(rows * 2 * H * 4)
    cal_src = cal_dst = None
    if args.calib:
        cal_src, cal_dst = DevBuf(256 << 20), DevBuf(256 << 20)

    sp = C.c_void_p()
    _lib.call("asca_stream_create", C.byref(sp))
    stream = sp.value
    V = lambda b: C.c_void_p(b.ptr)  # noqa: E731

    def fwd():
        _lib.call("asca_delta_fwd", V(dev["q"]), V(dev["k"]), V(dev["v"]), V(dev["alpha"]), V(dev["beta"]), V(o),
                  V(ws), B, T, H, dh, C.c_void_p(stream))

    def bwd():
        _lib.call("asca_delta_bwd_fused", V(dev["q"]), V(dev["k"]), V(dev["v"]), V(dev["alpha"]),
                  V(dev["beta"]), V(dev["qn"]), V(dev["kn"]), V(dev["d_o"]), V(ws), V(d_qkv), V(d_gate),
                  B, T, H, dh, C.c_void_p(stream))

    def event():
        e = C.c_void_p()
        _lib.call("asca_event_create", C.byref(e))
        return e

    def elapsed(a, b):
        ms = C.c_float()
        _lib.call("asca_event_elapsed_ms", C.byref(ms), a, b)
        return ms.value

    print(f"bench: {gpu.describe()}; B{B} T{T} H{H} dh{dh}; warmup {args.warmup}, steps {args.steps}", flush=True)
    # Bring the GPU to steady clocks first: a fresh box's first milliseconds of
    # matrix work run slower (the backward's first launches in a process take
    # ~15% longer than later ones).  The same fwd + bwd for a fixed wall time,
    # untimed, before the W warm-up steps; the timed region is unchanged.
    pw0 = time.perf_counter()
    n_pre = 0
    while time.perf_counter() - pw0 < args.prewarm_ms * 1e-3:
        for _ in range(10):
            fwd()
            bwd()
        n_pre += 10
        _lib.call("asca_stream_sync", C.c_void_p(stream))
    prewarm_ms = (time.perf_counter() - pw0) * 1e3
    for _ in range(args.warmup):
        fwd()
        bwd()
        if cal_src is not None:
            _lib.call("asca_copy_f32", V(cal_dst), V(cal_src), C.c_size_t((256 << 20) // 4), C.c_void_p(stream))
    _lib.call("asca_stream_sync", C.c_void_p(stream))

    K = args.steps
    # The timed region: K steps with a HIP event at each end and nothing else on
    # the stream (an event record between kernels costs ~3 us of stream time,
    # about 5% of a step, so the per-kernel events are in their own pass below).
    e_start, e_end = event(), event()
    t0 = time.perf_counter()
    _lib.call("asca_event_record", e_start, C.c_void_p(stream))
    for i in range(K):
        fwd()
        bwd()
    _lib.call("asca_event_record", e_end, C.c_void_p(stream))
    _lib.call("asca_stream_sync", C.c_void_p(stream))
    wall = time.perf_counter() - t0
    dev_ms = elapsed(e_start, e_end) / K
    # Kernel timing pass, right after on the same stream and inputs: the same K
    # steps with an event before and after each launch, for each kernel's
    # duration (the roofline's `achieved`).
    ev = [(event(), event(), event()) for _ in range(K)]
    for i in range(K):
        _lib.call("asca_event_record", ev[i][0], C.c_void_p(stream))
        fwd()
        _lib.call("asca_event_record", ev[i][1], C.c_void_p(stream))
        bwd()
        _lib.call("asca_event_record", ev[i][2], C.c_void_p(stream))
    _lib.call("asca_stream_sync", C.c_void_p(stream))
    fwd_ms = statistics.mean(elapsed(e[0], e[1]) for e in ev)
    bwd_ms = statistics.mean(elapsed(e[1], e[2]) for e in ev)
    for h in [e_start, e_end] + [h for e in ev for h in e]:
        _lib.call("asca_event_destroy", h)
    print(f"bench: device step {dev_ms:.4f} ms, wall step {wall / K * 1e3:.4f} ms (timed region); "
          f"kernel pass: fwd {fwd_ms:.4f} ms, bwd {bwd_ms:.4f} ms", flush=True)

    f_fwd, f_bwd, b_fwd, b_bwd = work_model(B, T, H, dh)
    step_s = wall / K
    tokens = B * T
    dominant = "delta_bwd" if bwd_ms >= fwd_ms else "delta_fwd"
    dom_ms = max(bwd_ms, fwd_ms)
    dom_f = f_bwd if dominant == "delta_bwd" else f_fwd
    dom_b = b_bwd if dominant == "delta_bwd" else b_fwd
    achieved = dom_f / (dom_ms * 1e-3)
    # HBM bytes per launch from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes, when
    # they were taken on the current kernel sources (else null: never stale)
    traffic, traffic_note = None, "no counter file"
    if PMC_FILE.exists():
        try:
            pmc = json.loads(PMC_FILE.read_text())
            if pmc.get("sources_sha") == kernel_sources_sha():
                traffic = pmc.get(dominant, {}).get("hbm_bytes_per_launch")
                traffic_note = "rocprofv3 FETCH_SIZE/WRITE_SIZE on these sources, calibrated by a copy kernel"
            else:
                traffic_note = "counters predate the current kernel sources"
        except (ValueError, OSError):
            traffic_note = "unreadable counter file"
    roof_step = max((f_fwd + f_bwd) / PEAK_F32, (b_fwd + b_bwd) / PEAK_HBM)
    result = {
        "metric": METRIC,
        "value": round(tokens / step_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "prewarm_ms": round(prewarm_ms, 1),
        "prewarm_steps": n_pre,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (reference Rng stream, configs[1] distributions, seed 1)",
        "config": {"workload": "gated delta-rule fwd+BPTT (asca_delta_fwd + asca_delta_bwd_fused): the recurrence "
                               "over T, state per (sequence, head) in registers, 16 steps per f32 MFMA block",
                   "B": B, "T": T, "H": H, "dh": dh, "seed": seed},
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved / 1e12, 3),
            "peak": PEAK_F32 / 1e12,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_F32, 4),
            "traffic": traffic,
            "traffic_note": traffic_note,
            "note": "achieved = the reference's algorithmic flops (17 dh^2 per token-head for the backward, "
                    "7 dh^2 forward) over the kernel time; the state recurrence and every product run on "
                    "the f32 matrix cores (v_mfma_f32_16x16x4_f32), 157.3 TFLOP/s dense peak",
            "kernel": dominant,
            "algorithmic_bytes": dom_b,
            "algorithmic_flops": dom_f,
        },
        "kernels_ms": {"delta_fwd": round(fwd_ms, 4), "delta_bwd": round(bwd_ms, 4)},
        "timing": "value and ms_per_step: host wall clock over the K timed steps (stream synchronised on "
                  "both sides; HIP events only at the region's ends); kernels_ms and roofline.achieved: HIP "
                  "events around each launch in a second pass of K steps right after it, on the same stream",
        "step_roofline": {
            "roofline_us": round(roof_step * 1e6, 2),
            "measured_us": round(dev_ms * 1e3, 2),
            "frac": round(roof_step / (dev_ms * 1e-3), 4),
            "note": "whole fwd+BPTT vs max(24 dh^2 flops / 157.3 TFLOP/s, compulsory bytes / 8 TB/s)",
        },
    }
    if not args.no_cpu:
        print("bench: timing the CPU baseline ...", flush=True)
        result["cpu_baseline"] = cpu_baseline(x, B, T, H, dh)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
