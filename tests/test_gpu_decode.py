"""GPU parity of the batched decode step (DeltaBlock::step state math,
rust/src/delta.rs:356-407) against the CPU oracle, through the C ABI."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _inputs(rng, n, H, dh):
    d = H * dh
    qkv = rng.standard_normal((n, 3 * d)).astype(np.float32)
    gate = rng.standard_normal((n, 2 * H)).astype(np.float32)
    gate[:, :H] += 2.0
    return qkv, gate


@pytest.mark.parametrize("n,H,dh,steps", [
    (3, 2, 8, 10),        # shape of the float64 golden
    (5, 4, 16, 12),
    (7, 3, 64, 8),        # the reference's cap
    (4, 2, 128, 6),       # beyond the reference's cap (configs[4] head size)
    (3, 2, 36, 5),        # dh % 4 == 0, not a power of two
    (2, 3, 50, 5),        # scalar path
])
def test_decode_steps_match_oracle(orc, g, n, H, dh, steps):
    print(f"[decode parity] n={n} H={H} dh={dh} steps={steps}", flush=True)
    rng = np.random.default_rng(n * 1000 + dh)
    S_ref = np.zeros((n, H, dh, dh), dtype=np.float32)
    S_dev = g.new_decode_states(n, H, dh)
    worst = 0.0
    for _ in range(steps):
        qkv, gate = _inputs(rng, n, H, dh)
        o_ref = orc.delta_decode_step(S_ref, qkv, gate, H, dh)
        o = g.delta_decode_step(S_dev, qkv, gate, H, dh)
        worst = max(worst, orc.rel_err(o, o_ref))
    S = S_dev.to_host((n, H, dh, dh))
    print(f"[decode parity] worst o rel {worst:.2e}, state rel {orc.rel_err(S, S_ref):.2e}", flush=True)
    assert worst <= 2e-5
    assert orc.rel_err(S, S_ref) <= 2e-5


def test_decode_config4_shape(orc, g):
    # 512 sequences, H=16, dh=128, seed 3 (a few steps here)
    n, H, dh = 512, 16, 128
    rng = np.random.default_rng(3)
    S_ref = np.zeros((n, H, dh, dh), dtype=np.float32)
    S_dev = g.new_decode_states(n, H, dh)
    for step in range(3):
        qkv, gate = _inputs(rng, n, H, dh)
        o_ref = orc.delta_decode_step(S_ref, qkv, gate, H, dh)
        o = g.delta_decode_step(S_dev, qkv, gate, H, dh)
        e = orc.rel_err(o, o_ref)
        print(f"[decode parity] configs[4] step {step} o rel {e:.2e}", flush=True)
        assert e <= 2e-5
    assert orc.rel_err(S_dev.to_host((n, H, dh, dh)), S_ref) <= 2e-5


def test_decode_config4_all_steps(orc, g):
    """configs[4] over its whole run: 512 sequences, H=16, dh=128, 256 steps,
    seed 3, all decoded on the GPU; every 16th sequence is followed by the
    oracle (the sequences are independent), its outputs at every step and its
    states at the end."""
    n, H, dh, steps = 512, 16, 128, 256
    sub = np.arange(0, n, 16)
    rng = np.random.default_rng(3)
    S_ref = np.zeros((sub.size, H, dh, dh), dtype=np.float32)
    S_dev = g.new_decode_states(n, H, dh)
    worst = 0.0
    for step in range(steps):
        qkv, gate = _inputs(rng, n, H, dh)
        o = g.delta_decode_step(S_dev, qkv, gate, H, dh)
        o_ref = orc.delta_decode_step(S_ref, np.ascontiguousarray(qkv[sub]), np.ascontiguousarray(gate[sub]), H, dh)
        worst = max(worst, orc.rel_err(o[sub], o_ref))
        if step % 64 == 63:
            print(f"[decode parity] configs[4] step {step + 1}/{steps}: worst o rel {worst:.2e}", flush=True)
    assert worst <= 2e-5
    S = S_dev.to_host((n, H, dh, dh))
    assert orc.rel_err(S[sub], S_ref) <= 2e-5


def test_decode_equals_forward_on_gpu(orc, g):
    # rust/tests/decode_parity.rs on the GPU path: token-by-token decode steps
    # reproduce the forward scan's outputs (rel <= 1e-4)
    T, H, dh = 24, 2, 32
    d = H * dh
    rng = np.random.default_rng(17)
    qkv, gate = _inputs(rng, T, H, dh)
    q, _ = orc.l2norm_heads(qkv[:, :d], H, dh)
    k, _ = orc.l2norm_heads(qkv[:, d:2 * d], H, dh)
    v = np.ascontiguousarray(qkv[:, 2 * d:])
    a = (1 / (1 + np.exp(-gate[:, :H]))).astype(np.float32)
    b = (1 / (1 + np.exp(-gate[:, H:]))).astype(np.float32)
    o_fwd, _ = g.delta_scan(q, k, v, a, b, 1, T, H, dh)
    S_dev = g.new_decode_states(1, H, dh)
    o_dec = np.concatenate([g.delta_decode_step(S_dev, qkv[t:t + 1].copy(), gate[t:t + 1].copy(), H, dh)
                            for t in range(T)])
    assert orc.rel_err(o_dec, o_fwd) <= 1e-4
