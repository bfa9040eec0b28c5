"""CPU checks of the fused activation producers: the oracle's rms_norm and gated activation pinned by
closed forms and invariants (the reference's own tests hold no vectors for them), and the C ABI's argument checks of
kf_hip_rms_norm_q8 / kf_hip_gated_act_q8 (rejected before any HIP call)."""
import math

import numpy as np
import pytest

import kungfu_amd as kf
import oracle


def _rms_norm_ieee(x, w=None, b=None, eps=1e-5):
    """ops::rms_norm (crates/kf-backend-cpu/src/ops.rs:222-239) with numpy's IEEE f32 operations: f32 squares summed
    in f64 (pairwise here, sequential in the oracle: the f32 result agrees), f32 sqrt and division."""
    x = x.astype(np.float32)
    out = np.empty_like(x)
    for r in range(x.shape[0]):
        ss = np.float32(np.sum((x[r] * x[r]).astype(np.float64)) / x.shape[1])
        inv = np.float32(1.0) / np.sqrt(ss + np.float32(eps))
        v = x[r] * inv
        v = v * (np.float32(1.0) if w is None else w.astype(np.float32))
        out[r] = v + (np.float32(0.0) if b is None else b.astype(np.float32))
    return out


@pytest.mark.parametrize("n", [32, 4096, 14336])
def test_rms_norm_matches_ieee_restatement(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((3, n)) * rng.uniform(0.01, 30, (3, 1))).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    assert np.array_equal(oracle.rms_norm(x, w, b, 1e-6), _rms_norm_ieee(x, w, b, 1e-6))
    assert np.array_equal(oracle.rms_norm(x), _rms_norm_ieee(x))


def test_rms_norm_invariants():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 1024)).astype(np.float32)
    # unit weight, no bias: the output's mean square is ss / (ss + eps)
    eps = 0.25
    y = oracle.rms_norm(x, eps=eps).astype(np.float64)
    ss = (x.astype(np.float64) ** 2).mean(axis=1)
    assert np.allclose((y ** 2).mean(axis=1), ss / (ss + eps), rtol=1e-6)
    # with eps = 0 the norm is invariant, bit for bit, under power-of-two scaling (every step scales exactly)
    for k in (-20, -3, 5, 30):
        assert np.array_equal(oracle.rms_norm(x * np.float32(2.0**k), eps=0.0), oracle.rms_norm(x, eps=0.0))
    # a constant row c: every value is c / sqrt(c^2 + eps) * w + b
    c = np.full((1, 64), -3.0, np.float32)
    w = np.linspace(-2, 2, 64).astype(np.float32)
    got = oracle.rms_norm(c, w, np.ones(64, np.float32), 1e-3)
    want = np.float32(-3.0) * (np.float32(1.0) / np.sqrt(np.float32(9.0) + np.float32(1e-3))) * w + np.float32(1.0)
    assert np.array_equal(got[0], want)
    # weight and bias are applied per column: a zero weight leaves the bias
    assert np.array_equal(oracle.rms_norm(x, np.zeros(1024, np.float32), np.full(1024, 7.0, np.float32)), np.full_like(x, 7.0))


def test_silu_and_gated_closed_forms():
    assert oracle.silu(0.0) == 0.0
    assert oracle.silu(100.0) == 100.0          # exp(-100) is below half an ulp of 1
    assert oracle.silu(-200.0) == 0.0           # exp(200) overflows f32: -200 / inf = -0
    for v in np.linspace(-12, 12, 97):
        # silu(x) - silu(-x) = x; sigma from the f64 definition within a few ulps
        s, t = oracle.silu(v), oracle.silu(-v)
        assert abs((s - t) - v) <= 4e-6 * max(1.0, abs(v))
        assert math.isclose(s, v / (1.0 + math.exp(-v)), rel_tol=2e-7, abs_tol=1e-30)
    rng = np.random.default_rng(2)
    g = rng.standard_normal((3, 2 * 64)).astype(np.float32) * 4
    # gate and up side by side in one row (stride 2n)
    gate, up = g[:, :64], g[:, 64:]
    relu = oracle.gated(kf.GLU_RELU, g.ravel(), g.ravel()[64:], 3, 64, 128)
    assert np.array_equal(relu, np.maximum(gate, 0) * up)
    sq = oracle.gated(kf.GLU_RELU_SQR, g.ravel(), g.ravel()[64:], 3, 64, 128)
    assert np.array_equal(sq, (np.maximum(gate, 0) * np.maximum(gate, 0)) * up)
    si = oracle.gated(kf.GLU_SILU, gate.copy(), up.copy(), 3, 64, 64)
    assert np.array_equal(si, np.array([[oracle.silu(a) for a in r] for r in gate], np.float32) * up)


FAKE = 0x10000  # a 256-byte aligned address the checks must reject before any HIP call


def _rc(fn, *args):
    rc = fn(*args)
    return rc, kf.last_error() if rc < 0 else ""


def test_producer_argument_checks():
    L = kf.lib()
    rms, glu = L.kf_hip_rms_norm_q8, L.kf_hip_gated_act_q8
    rc, msg = _rc(rms, FAKE, None, None, 1, 4096, 1e-5, 5, FAKE, None)
    assert rc == kf.KF_E_UNSUPPORTED and "kind 5" in msg
    rc, msg = _rc(rms, FAKE, None, None, 1, 100, 1e-5, kf.ACT_Q8_0, FAKE, None)
    assert rc == kf.KF_E_INVALID and "100 columns" in msg
    rc, msg = _rc(rms, FAKE, None, None, 1, 4096, 1e-5, kf.ACT_Q8K, FAKE + 64, None)
    assert rc == kf.KF_E_INVALID and "256-byte" in msg
    rc, msg = _rc(rms, FAKE + 4, None, None, 1, 4096, 1e-5, kf.ACT_Q8K, FAKE, None)
    assert rc == kf.KF_E_INVALID and "16-byte" in msg
    rc, msg = _rc(rms, FAKE, FAKE + 8, None, 1, 4096, 1e-5, kf.ACT_Q8K, FAKE, None)
    assert rc == kf.KF_E_INVALID and "16-byte" in msg
    rc, msg = _rc(rms, FAKE, None, None, 1, 4096, -1.0, kf.ACT_Q8K, FAKE, None)
    assert rc == kf.KF_E_INVALID and "eps" in msg
    rc, msg = _rc(glu, FAKE, FAKE, 1, 256, 512, 1, kf.ACT_Q8_0, FAKE, None)
    assert rc == kf.KF_E_UNSUPPORTED and "activation 1" in msg
    rc, msg = _rc(glu, FAKE, FAKE, 1, 256, 128, kf.GLU_SILU, kf.ACT_Q8_0, FAKE, None)
    assert rc == kf.KF_E_INVALID and "stride 128" in msg
    rc, msg = _rc(glu, FAKE, FAKE + 4, 1, 256, 512, kf.GLU_SILU, kf.ACT_Q8_0, FAKE, None)
    assert rc == kf.KF_E_INVALID and "16-byte" in msg
    rc, msg = _rc(glu, FAKE, FAKE, 0, 256, 512, kf.GLU_SILU, kf.ACT_Q8_0, FAKE, None)
    assert rc == kf.KF_E_INVALID and "0 rows" in msg
