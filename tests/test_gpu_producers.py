"""GPU parity of the fused activation producers (kf_hip_rms_norm_q8, kf_hip_gated_act_q8) through the C ABI: the
int8 values, per-16/32 scales and integer sums equal the oracle's quantize_activations of the oracle's rms_norm /
gated activation (the CPU backend's values), bit for bit."""
import numpy as np
import pytest

import kungfu_amd as kf
import oracle

pytestmark = pytest.mark.gpu


def _tensor(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _check_act(act, rows, n, kind, values):
    import torch

    torch.cuda.synchronize()
    q, d16, s16, d32, s32 = [t.cpu().numpy() for t in kf.act_views(act, rows, n)]
    wq, wd, ws = oracle.quantize_activations(kind, values)
    assert np.array_equal(q, wq), f"{(q != wq).sum()} of {q.size} int8 values differ"
    assert np.array_equal(d16.view(np.uint32), wd.view(np.uint32))
    assert np.array_equal(s16, ws)
    assert np.array_equal(d32.view(np.uint32), wd[:, ::2].view(np.uint32))
    assert np.array_equal(s32, ws[:, ::2] + ws[:, 1::2])


@pytest.mark.parametrize("kind", [kf.ACT_Q8_0, kf.ACT_Q8K])
@pytest.mark.parametrize("rows,n,affine", [(1, 4096, True), (3, 256, False), (7, 14336, True), (33, 4096, False), (2, 20480, True),
                                          (70, 4096, True), (70, 14336, False)])
def test_rms_norm_q8_bit_exact(cuda, kind, rows, n, affine):
    rng = np.random.default_rng(rows * 7 + n + kind)
    x = (rng.standard_normal((rows, n)) * rng.uniform(0.01, 40, (rows, 1))).astype(np.float32)
    x[0, :256] = 0.0  # an all-zero block inside a nonzero row
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32) if affine else None
    b = (0.01 * rng.standard_normal(n)).astype(np.float32) if affine else None
    eps = 1e-5
    act = kf.alloc_act(rows, n, cuda)
    kf.rms_norm_q8(_tensor(x, cuda), act, kind, None if w is None else _tensor(w, cuda), None if b is None else _tensor(b, cuda), eps)
    _check_act(act, rows, n, kind, oracle.rms_norm(x, w, b, eps))


def test_rms_norm_q8_zero_row(cuda):
    """An all-zero row with eps = 0 divides by zero in the CPU too (inf * 0 = nan): with eps > 0 it quantizes to zeros."""
    x = np.zeros((2, 512), np.float32)
    x[1] = np.linspace(-1, 1, 512, dtype=np.float32)
    act = kf.alloc_act(2, 512, cuda)
    kf.rms_norm_q8(_tensor(x, cuda), act, kf.ACT_Q8K, eps=1e-6)
    _check_act(act, 2, 512, kf.ACT_Q8K, oracle.rms_norm(x, eps=1e-6))


@pytest.mark.parametrize("act_fn", [kf.GLU_SILU, kf.GLU_RELU, kf.GLU_RELU_SQR])
@pytest.mark.parametrize("kind", [kf.ACT_Q8_0, kf.ACT_Q8K])
@pytest.mark.parametrize("rows,n", [(1, 14336), (5, 256), (16, 4096)])
def test_gated_act_q8_fused_rows_bit_exact(cuda, act_fn, kind, rows, n):
    """gate and up as the two halves of one fused gate+up output row (stride 2n), as the gate+up product writes them."""
    rng = np.random.default_rng(rows + n + act_fn * 11 + kind)
    gu = (rng.standard_normal((rows, 2 * n)) * 3).astype(np.float32)
    gu[0, :32] = 0.0
    gu[-1, 40] = -120.0  # silu far below zero: exp overflows to inf, the value is -0
    t = _tensor(gu, cuda)
    act = kf.alloc_act(rows, n, cuda)
    kf.gated_act_q8(t[:, :n], t[:, n:], act, kind, rows, n, 2 * n, act_fn)
    _check_act(act, rows, n, kind, oracle.gated(act_fn, gu.ravel(), gu.ravel()[n:], rows, n, 2 * n))


def test_gated_act_q8_separate_tensors(cuda):
    rng = np.random.default_rng(9)
    rows, n = 4, 4096
    g = (rng.standard_normal((rows, n)) * 6).astype(np.float32)
    u = rng.standard_normal((rows, n)).astype(np.float32)
    act = kf.alloc_act(rows, n, cuda)
    kf.gated_act_q8(_tensor(g, cuda), _tensor(u, cuda), act, kf.ACT_Q8K, rows, n, n, kf.GLU_SILU)
    _check_act(act, rows, n, kf.ACT_Q8K, oracle.gated(kf.GLU_SILU, g, u, rows, n, n))


def test_producer_feeds_the_product(cuda):
    """rms_norm_q8 then the GEMV equals the CPU backend's rms_norm followed by matmul_slice (the f32 bar)."""
    import torch

    rng = np.random.default_rng(5)
    n, n_out = 4096, 512
    x = rng.standard_normal((1, n)).astype(np.float32)
    w_norm = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    wq = kf.quantize(kf.TYPE_Q4_K, kf.synth_normal(3, 0.02, n * n_out).reshape(n_out, n))
    act = kf.alloc_act(1, n, cuda)
    kf.rms_norm_q8(_tensor(x, cuda), act, kf.ACT_Q8K, _tensor(w_norm, cuda), None, 1e-5)
    y = torch.empty((1, n_out), device=cuda)
    kf.gemv(kf.TYPE_Q4_K, _tensor(wq, cuda), act, y, 1, n, n_out)
    torch.cuda.synchronize()
    want = oracle.matmul_slice(kf.TYPE_Q4_K, wq, n, n_out, oracle.rms_norm(x, w_norm, None, 1e-5))
    err = np.abs(y.cpu().numpy() - want)
    assert (err <= 1e-4 + 1e-3 * np.abs(want)).all(), err.max()


@pytest.mark.parametrize("ty", [kf.TYPE_Q4_K, kf.TYPE_Q8_0])
@pytest.mark.parametrize("rows,n,n_out,affine", [(1, 4096, 520, True), (1, 2048, 300, False), (1, 256, 64, True), (1, 4096, 6144, False),
                                                 (1, 3584, 96, True), (3, 4096, 200, True)])
def test_rms_norm_matmul(cuda, knobs, ty, rows, n, n_out, affine):
    """kf_hip_rms_norm_matmul: at one row the GEMV normalises and quantizes the row in every block (one launch),
    bit-identical to kf_hip_rms_norm_q8 followed by the product (KF_MATMUL_NO_FUSE); both against the CPU backend's
    matmul_slice of its rms_norm. Three rows take the two-launch path. Widths of one to sixteen 256-column chunks
    (some waves of a block hold no chunk)."""
    import torch

    rng = np.random.default_rng(n + n_out + ty)
    x = (rng.standard_normal((rows, n)) * rng.uniform(0.05, 30, (rows, 1))).astype(np.float32)
    wn = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32) if affine else None
    bn = (0.01 * rng.standard_normal(n)).astype(np.float32) if affine else None
    w = kf.quantize(ty, kf.synth_normal(n + 3, 0.02, n * n_out).reshape(n_out, n))
    bias = kf.synth_normal(5, 1.0, n_out)
    res = kf.synth_normal(6, 1.0, rows * n_out).reshape(rows, n_out)
    wt, xt, bt, rt = (_tensor(a, cuda) for a in (w, x, bias, res))
    wnt = None if wn is None else _tensor(wn, cuda)
    bnt = None if bn is None else _tensor(bn, cuda)
    act = kf.alloc_act(rows, n, cuda)
    outs = []
    for fuse in (True, False):
        if fuse:
            knobs.delenv("KF_MATMUL_NO_FUSE", raising=False)
        else:
            knobs.setenv("KF_MATMUL_NO_FUSE", "1")
        y = torch.full((rows, n_out), float("nan"), device=cuda)
        kf.rms_norm_matmul(ty, wt, xt, act, y, n_out, wnt, bnt, 1e-5, bias=bt, res=rt)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    want = oracle.matmul_slice(ty, w, n, n_out, oracle.rms_norm(x, wn, bn, 1e-5), bias) + res
    err = np.abs(outs[0].astype(np.float64) - want)
    assert (err <= 1e-4 + 1e-3 * np.abs(want)).all(), f"max error {err.max():.3e}"
