"""Calls from several host threads at once, in a fresh process, so that the
first launches of each kernel (where the library allows a kernel its dynamic
LDS on the device, once per kernel and device, under a lock) race: every
thread's result must equal the same call made again alone, bit for bit.
All calls go through the C ABI (asca_amd.gpu -> libasca_hip.so).
"""
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

SCRIPT = textwrap.dedent("""
    import sys, threading
    import numpy as np
    sys.path.insert(0, sys.argv[1])
    from asca_amd import gpu

    g = gpu.gpu()
    assert g is not None, gpu.describe()
    B, T, H, dh = 2, 40, 2, 64

    def inputs(seed):
        r = np.random.default_rng(seed)
        rows, d = B * T, H * dh
        q = r.standard_normal((rows, d), dtype=np.float32)
        k = r.standard_normal((rows, d), dtype=np.float32)
        for x in (q, k):
            x3 = x.reshape(rows, H, dh)
            x3 /= np.linalg.norm(x3, axis=2, keepdims=True)
        v = r.standard_normal((rows, d), dtype=np.float32)
        a = (1 / (1 + np.exp(-(2 + r.standard_normal((rows, H)))))).astype(np.float32)
        b = (1 / (1 + np.exp(-r.standard_normal((rows, H))))).astype(np.float32)
        d_o = r.standard_normal((rows, d), dtype=np.float32)
        ga = r.standard_normal((96, 160), dtype=np.float32)
        gb = r.standard_normal((160, 72), dtype=np.float32)
        return q, k, v, a, b, d_o, ga, gb

    def run(x):
        q, k, v, a, b, d_o, ga, gb = x
        o, dev = g.delta_scan(q, k, v, a, b, B, T, H, dh)
        dq, dk, dv, da, db = g.delta_bwd_raw(dev, d_o)
        return [o, dq, dk, dv, da, db, g.matmul(ga, gb)]

    xs = [inputs(s) for s in range(4)]
    got = [None] * 4
    errs = []
    start = threading.Barrier(4)

    def worker(i):
        try:
            start.wait()
            got[i] = run(xs[i])
        except BaseException as e:  # reported by the main thread
            errs.append(repr(e))

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errs, errs
    for i in range(4):
        want = run(xs[i])
        for a, b in zip(got[i], want):
            np.testing.assert_array_equal(a, b)
    print("threads ok", flush=True)
""")


def test_first_calls_from_four_threads():
    print("[threads] four host threads, first launches of delta fwd/bwd and GEMM", flush=True)
    r = subprocess.run([sys.executable, "-c", SCRIPT, str(ROOT)], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "threads ok" in r.stdout
