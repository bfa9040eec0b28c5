"""GPU parity of the HIP path against the CPU oracle, called through the C ABI on the same seeded inputs.

Bar (from the north star): per-block int32 results bit-exact; fp32 outputs within |got - want| <= 1e-4 + 1e-3 * |want|
of kf-backend-cpu's matmul_slice (crates/kf-backend-cpu/src/ops.rs:304-346); the quantized activations bit-exact with
quantize_activations (crates/kf-quant/src/lib.rs:81-140). Shapes follow the reference's differential tests
(crates/kf-backend-cuda/tests/quant.rs:46-83: ragged n_out, several widths) plus the full Llama-3-8B shapes.
"""
import numpy as np
import pytest

import kungfu_amd as kf
import oracle

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4


def _tensor(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _weights(ty, n_out, n_in, seed):
    w = kf.synth_normal(seed, 0.02, n_out * n_in).reshape(n_out, n_in)
    return kf.quantize(ty, w)


def _close(got, want):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bad = err > ATOL + RTOL * np.abs(want)
    assert not bad.any(), f"{bad.sum()} outputs off, worst {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"


@pytest.mark.parametrize("kind", [kf.ACT_Q8_0, kf.ACT_Q8K])
@pytest.mark.parametrize("rows,n", [(1, 256), (3, 4096), (2, 14336), (5, 1024)])
def test_quant_act_bit_exact(cuda, kind, rows, n):
    import torch

    rng = np.random.default_rng(rows * 100 + n + kind)
    x = (rng.standard_normal((rows, n)) * rng.uniform(1e-3, 50, (rows, 1))).astype(np.float32)
    x[0, :256] = 0.0                       # an all-zero block
    if n >= 512:
        x[-1, 256:288] = 2.5               # ties inside a block
        x[-1, 300] = -np.abs(x[-1, 256:512]).max() * 1.5  # a negative maximum late in the block
    if n >= 1024:
        x[0, 512 + 7] = 9.0
        x[0, 512 + 100] = -9.0             # equal magnitudes: the first index sets the sign of the scale
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kind)
    torch.cuda.synchronize()
    q, d16, s16, d32, s32 = [t.cpu().numpy() for t in kf.act_views(act, rows, n)]
    wq, wd, ws = oracle.quantize_activations(kind, x)
    assert np.array_equal(q, wq)
    assert np.array_equal(d16.view(np.uint32), wd.view(np.uint32))
    assert np.array_equal(s16, ws)
    assert np.array_equal(d32.view(np.uint32), wd[:, ::2].view(np.uint32))
    assert np.array_equal(s32, ws[:, ::2] + ws[:, 1::2])
    if kind == kf.ACT_Q8K:
        # the mins operand: per 256 columns the eight per-32 sums as floor(s / 64), then s mod 64
        xa = kf.act_xa(act, rows, n).cpu().numpy().astype(np.float64)
        s32w = (ws[:, ::2] + ws[:, 1::2]).astype(np.int64).reshape(rows, n // 256, 8)
        assert np.array_equal(xa[:, :, :8], s32w // 64) and np.array_equal(xa[:, :, 8:], s32w % 64)


def test_quant_act_hard_rounding_ties(cuda):
    """Planted ties where the f32 product is k + 0.5 but the real product is below it (half of all elements)."""
    import torch
    from tie_inputs import hard_tie_rows

    x, made = hard_tie_rows(16, 1024, seed=3)
    assert made > 4000
    act = kf.alloc_act(16, 1024, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8_0)
    torch.cuda.synchronize()
    q = kf.act_views(act, 16, 1024)[0].cpu().numpy()
    wq, _, _ = oracle.quantize_activations(kf.ACT_Q8_0, x)
    assert np.array_equal(q, wq), f"{(q != wq).sum()} of {q.size} differ"


def _random_blocks(ty, n_out, n_in, rng):
    """Random block bytes with sane f16 scales (the harness of crates/kf-backend-cuda/tests/common/mod.rs:100-147)."""
    block, size = kf.BLOCK[ty]
    w = rng.integers(0, 256, (n_out, n_in // block, size), dtype=np.uint8)
    bits = (((5 + rng.integers(0, 8, w.shape[:2])) << 10) | rng.integers(0, 1024, w.shape[:2])).astype(np.uint16)
    w[:, :, 0:2] = bits.view(np.uint8).reshape(w.shape[0], w.shape[1], 2)
    if ty == kf.TYPE_Q4_K:
        bits = (((5 + rng.integers(0, 8, w.shape[:2])) << 10) | rng.integers(0, 1024, w.shape[:2])).astype(np.uint16)
        w[:, :, 2:4] = bits.view(np.uint8).reshape(w.shape[0], w.shape[1], 2)
    return w.reshape(n_out, -1)


@pytest.mark.parametrize("ty", [kf.TYPE_Q8_0, kf.TYPE_Q4_K])
@pytest.mark.parametrize("rows,n,n_out", [(1, 256, 5), (2, 1024, 7), (3, 4096, 3)])
def test_block_ints_bit_exact(cuda, ty, rows, n, n_out):
    import torch

    rng = np.random.default_rng(n + n_out + ty)
    w = _random_blocks(ty, n_out, n, rng)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.act_kind(ty))
    per = n // 32 if ty == kf.TYPE_Q8_0 else 2 * (n // 256)
    out = torch.zeros(n_out * rows * per, dtype=torch.int32, device=cuda)
    kf.block_ints(ty, _tensor(w, cuda), act, out, rows, n, n_out)
    got = out.cpu().numpy().reshape(n_out, rows, per)
    q, _, s16 = oracle.quantize_activations(kf.act_kind(ty), x)
    for o in range(n_out):
        for r in range(rows):
            assert np.array_equal(got[o, r], oracle.block_ints(ty, w[o], q[r], s16[r])), (o, r)


GEMV_SHAPES = [
    (kf.TYPE_Q4_K, 256, 1),
    (kf.TYPE_Q4_K, 256, 13),
    (kf.TYPE_Q4_K, 1024, 77),
    (kf.TYPE_Q4_K, 2304, 33),      # 9 super-blocks: a ragged wave step
    (kf.TYPE_Q4_K, 4096, 520),
    (kf.TYPE_Q4_K, 14336, 300),
    (kf.TYPE_Q4_K, 32768, 40),     # the widest row the GEMV stages
    (kf.TYPE_Q8_0, 32, 3),
    (kf.TYPE_Q8_0, 96, 11),        # odd block count: rows start 2 bytes into a dword
    (kf.TYPE_Q8_0, 2080, 17),
    (kf.TYPE_Q8_0, 4096, 515),
    (kf.TYPE_Q8_0, 14336, 64),
    (kf.TYPE_Q8_0, 32768, 9),
]


@pytest.mark.parametrize("ty,n,n_out", GEMV_SHAPES)
def test_gemv_matches_cpu_backend(cuda, ty, n, n_out):
    import torch

    w = _weights(ty, n_out, n, seed=n + n_out)
    x = kf.synth_normal(7 + n, 1.0, n).reshape(1, n)
    wd = _tensor(w, cuda)
    xd = _tensor(x, cuda)
    act = kf.alloc_act(1, n, cuda)
    y = torch.full((1, n_out), float("nan"), device=cuda)
    kf.matmul(ty, wd, xd, act, y, n_out)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    _close(got, oracle.matmul_slice(ty, w, n, n_out, x))
    # against the integer CPU path the only difference left is the order of float additions
    yi = oracle.matmul_i8(ty, w, n, n_out, x)
    assert np.abs(got - yi).max() <= 2e-5 * max(1.0, np.abs(yi).max())


LLAMA_SHAPES = [(4096, 6144), (4096, 4096), (4096, 14336), (4096, 28672), (14336, 4096)]


@pytest.mark.parametrize("n,n_out", LLAMA_SHAPES)
def test_gemv_q4_k_llama_shapes(cuda, n, n_out):
    import torch

    w = _weights(kf.TYPE_Q4_K, n_out, n, seed=0)
    x = kf.synth_normal(1, 1.0, n).reshape(1, n)
    act = kf.alloc_act(1, n, cuda)
    y = torch.empty((1, n_out), device=cuda)
    kf.matmul(kf.TYPE_Q4_K, _tensor(w, cuda), _tensor(x, cuda), act, y, n_out)
    torch.cuda.synchronize()
    _close(y.cpu().numpy(), oracle.matmul_slice(kf.TYPE_Q4_K, w, n, n_out, x))


def test_gemv_q8_0_config_c1(cuda):
    import torch

    n = n_out = 4096
    w = _weights(kf.TYPE_Q8_0, n_out, n, seed=0)
    x = kf.synth_normal(1, 1.0, n).reshape(1, n)
    act = kf.alloc_act(1, n, cuda)
    y = torch.empty((1, n_out), device=cuda)
    kf.matmul(kf.TYPE_Q8_0, _tensor(w, cuda), _tensor(x, cuda), act, y, n_out)
    torch.cuda.synchronize()
    _close(y.cpu().numpy(), oracle.matmul_slice(kf.TYPE_Q8_0, w, n, n_out, x))


@pytest.mark.parametrize("ty", [kf.TYPE_Q8_0, kf.TYPE_Q4_K])
def test_gemv_bias_and_residual(cuda, ty):
    import torch

    n, n_out = 1024, 96
    w = _weights(ty, n_out, n, seed=3)
    x = kf.synth_normal(4, 1.0, n).reshape(1, n)
    bias = kf.synth_normal(5, 1.0, n_out)
    res = kf.synth_normal(6, 1.0, n_out).reshape(1, n_out)
    act = kf.alloc_act(1, n, cuda)
    y = torch.empty((1, n_out), device=cuda)
    kf.matmul(ty, _tensor(w, cuda), _tensor(x, cuda), act, y, n_out, bias=_tensor(bias, cuda), res=_tensor(res, cuda))
    torch.cuda.synchronize()
    _close(y.cpu().numpy(), oracle.matmul_slice(ty, w, n, n_out, x, bias) + res)


@pytest.mark.parametrize("ty", [kf.TYPE_Q8_0, kf.TYPE_Q4_K])
@pytest.mark.parametrize("rows", [2, 3, 8])
def test_multi_row_matches_cpu_backend(cuda, ty, rows):
    import torch

    n, n_out = 2048, 130
    w = _weights(ty, n_out, n, seed=rows)
    x = kf.synth_normal(10 + rows, 1.0, rows * n).reshape(rows, n)
    act = kf.alloc_act(rows, n, cuda)
    y = torch.empty((rows, n_out), device=cuda)
    kf.matmul(ty, _tensor(w, cuda), _tensor(x, cuda), act, y, n_out)
    torch.cuda.synchronize()
    _close(y.cpu().numpy(), oracle.matmul_slice(ty, w, n, n_out, x))


def test_backend_mirror_matmul_and_slices(cuda):
    n, n_out, n_slices = 512, 48, 3
    w = _weights(kf.TYPE_Q4_K, n_out * n_slices, n, seed=21)
    x = kf.synth_normal(22, 1.0, 2 * n).reshape(2, n)
    bias = kf.synth_normal(23, 1.0, n_out)
    be = kf.Backend(0)
    try:
        wid = be.add_weight(kf.TYPE_Q4_K, [n, n_out, n_slices], w)
        _close(be.matmul(wid, x, n_out, bias), oracle.matmul_slice(kf.TYPE_Q4_K, w[:n_out], n, n_out, x, bias))
        for s in range(n_slices):
            got = be.matmul_slice(wid, s, x, n_out)
            _close(got, oracle.matmul_slice(kf.TYPE_Q4_K, w[s * n_out : (s + 1) * n_out], n, n_out, x))
        with pytest.raises(kf.KfError, match="columns against"):
            be.matmul(wid, x[:, :256], n_out)
        with pytest.raises(kf.KfError, match="slice 3 of 3"):
            be.matmul_slice(wid, 3, x, n_out)
    finally:
        be.close()


@pytest.mark.parametrize("dma", [True, False])
@pytest.mark.parametrize("maxit", ["1", "2", "4"])
@pytest.mark.parametrize("ty,n,n_out", [(kf.TYPE_Q4_K, 4096, 1030), (kf.TYPE_Q4_K, 14336, 77), (kf.TYPE_Q8_0, 4096, 777),
                                        (kf.TYPE_Q8_0, 14336, 45), (kf.TYPE_Q4_K, 32768, 9)])
def test_gemv_launch_variants(cuda, knobs, dma, maxit, ty, n, n_out):
    """Both GEMV kernels (direct-to-LDS and register-staged) at every row-iteration count agree with the CPU backend."""
    import torch

    knobs.setenv("KF_GEMV_MAXIT", maxit)
    if not dma:
        knobs.setenv("KF_GEMV_NO_DMA", "1")
    w = _weights(ty, n_out, n, seed=31)
    x = kf.synth_normal(32, 1.0, n).reshape(1, n)
    act = kf.alloc_act(1, n, cuda)
    y = torch.empty((1, n_out), device=cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.act_kind(ty))
    kf.gemv(ty, _tensor(w, cuda), act, y, 1, n, n_out)
    torch.cuda.synchronize()
    _close(y.cpu().numpy(), oracle.matmul_slice(ty, w, n, n_out, x))


@pytest.mark.parametrize("ty,n,n_out", [(kf.TYPE_Q4_K, 4096, 1030), (kf.TYPE_Q4_K, 4096, 6144), (kf.TYPE_Q8_0, 4096, 777),
                                        (kf.TYPE_Q4_K, 2304, 9)])
def test_gemv_one_shot_variant(cuda, knobs, ty, n, n_out):
    """The one-shot GEMV (every wave's row fetched straight into LDS at launch; KF_GEMV_ONESHOT=1, no longer the
    default for any shape) against the default persistent variant, bit for bit, and the CPU backend."""
    import torch

    w = _tensor(_weights(ty, n_out, n, seed=37), cuda)
    x = kf.synth_normal(38, 1.0, n).reshape(1, n)
    act = kf.alloc_act(1, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.act_kind(ty))
    outs = []
    for one_shot in (False, True):
        if one_shot:
            knobs.setenv("KF_GEMV_ONESHOT", "1")
        y = torch.full((1, n_out), float("nan"), device=cuda)
        kf.gemv(ty, w, act, y, 1, n, n_out)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    _close(outs[1], oracle.matmul_slice(ty, w.cpu().numpy(), n, n_out, x))


@pytest.mark.parametrize("ty,n,n_out", [(kf.TYPE_Q4_K, 4096, 4096), (kf.TYPE_Q4_K, 4096, 6144), (kf.TYPE_Q4_K, 4096, 28672),
                                        (kf.TYPE_Q4_K, 4096, 30000), (kf.TYPE_Q4_K, 14336, 4096), (kf.TYPE_Q4_K, 14336, 4100),
                                        (kf.TYPE_Q4_K, 2304, 9),
                                        (kf.TYPE_Q8_0, 4096, 4096), (kf.TYPE_Q8_0, 14336, 1030), (kf.TYPE_Q8_0, 4128, 77)])
def test_gemv_burst_variant(cuda, knobs, ty, n, n_out):
    """The burst GEMV (every wave's rows requested at launch, activation operands loaded per lane) forced at one to
    eight rows a wave and one to eight waves a row (KF_GEMV_BURST=8) against the pipelined kernel (KF_GEMV_BURST=0),
    bit for bit with bias and residual, and the CPU backend within the f32 bar. 14336 -> 4100: the pipelined kernel's
    split rows walk contiguous row ranges per block, the last ones partial or empty."""
    import torch

    w = _tensor(_weights(ty, n_out, n, seed=47), cuda)
    x = kf.synth_normal(48, 1.0, n).reshape(1, n)
    bias = _tensor(kf.synth_normal(49, 1.0, n_out), cuda)
    res = _tensor(kf.synth_normal(50, 1.0, n_out).reshape(1, n_out), cuda)
    act = kf.alloc_act(1, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.act_kind(ty))
    outs = []
    for rows in ("0", "8"):
        knobs.setenv("KF_GEMV_BURST", rows)
        y = torch.full((1, n_out), float("nan"), device=cuda)
        kf.gemv(ty, w, act, y, 1, n, n_out, bias=bias, res=res)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    want = oracle.matmul_slice(ty, w.cpu().numpy(), n, n_out, x) + bias.cpu().numpy() + res.cpu().numpy()
    _close(outs[1], want)


@pytest.mark.parametrize("ty,n,n_out", [(kf.TYPE_Q4_K, 256, 40), (kf.TYPE_Q4_K, 1280, 300), (kf.TYPE_Q4_K, 4096, 1030),
                                        (kf.TYPE_Q4_K, 2304, 777), (kf.TYPE_Q4_K, 14336, 64),
                                        (kf.TYPE_Q8_0, 32, 7), (kf.TYPE_Q8_0, 1056, 300), (kf.TYPE_Q8_0, 4096, 777),
                                        (kf.TYPE_Q8_0, 2080, 45), (kf.TYPE_Q8_0, 4128, 9)])
def test_matmul_one_row_fused_equals_two_launches(cuda, knobs, ty, n, n_out):
    """kf_hip_matmul at one row quantizes inside the GEMV (one launch; up to 4096 columns, past that the two launches):
    the same integers and scales as quant_act, so its outputs equal quant_act + kf_hip_gemv bit for bit, with bias and
    residual, on a row with an all-zero block, ties and a negative maximum; and the CPU backend's within the f32 bar."""
    import torch

    rng = np.random.default_rng(n + n_out)
    w = _weights(ty, n_out, n, seed=41)
    x = (rng.standard_normal((1, n)) * rng.uniform(0.01, 20)).astype(np.float32)
    x[0, : min(n, 256)] = 0.0
    if n >= 512:
        x[0, 256:288] = 1.5
        x[0, 300] = -np.abs(x[0, 256:512]).max() * 1.25
    bias = kf.synth_normal(42, 1.0, n_out)
    res = kf.synth_normal(43, 1.0, n_out).reshape(1, n_out)
    wt, xt, bt, rt = (_tensor(a, cuda) for a in (w, x, bias, res))
    act = kf.alloc_act(1, n, cuda)
    y1 = torch.full((1, n_out), float("nan"), device=cuda)
    kf.matmul(ty, wt, xt, act, y1, n_out, bias=bt, res=rt)
    y2 = torch.full((1, n_out), float("nan"), device=cuda)
    kf.quant_act(xt, act, kf.act_kind(ty))
    kf.gemv(ty, wt, act, y2, 1, n, n_out, bias=bt, res=rt)
    knobs.setenv("KF_MATMUL_NO_FUSE", "1")
    y3 = torch.full((1, n_out), float("nan"), device=cuda)
    kf.matmul(ty, wt, xt, act, y3, n_out, bias=bt, res=rt)
    torch.cuda.synchronize()
    got = y1.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), y2.cpu().numpy().view(np.uint32))
    assert np.array_equal(got.view(np.uint32), y3.cpu().numpy().view(np.uint32))
    _close(got, oracle.matmul_slice(ty, w, n, n_out, x, bias) + res)


GEMM_SHAPES = [(2, 128, 64), (9, 1024, 1000), (130, 512, 200), (256, 4096, 384), (64, 14336, 96), (8, 14336, 520),
               (33, 4096, 300), (48, 2048, 136), (16, 4096, 4096), (64, 4096, 4160),
               (1, 512, 40), (65, 1024, 130)]


@pytest.mark.parametrize("rows,n,n_out", GEMM_SHAPES)
def test_gemm_matches_cpu_backend(cuda, rows, n, n_out):
    """The int8 MFMA GEMM (q8_0) against matmul_slice; ragged row and column counts exercise the tile edges."""
    import torch

    w = _weights(kf.TYPE_Q8_0, n_out, n, seed=40 + rows)
    x = kf.synth_normal(41 + rows, 1.0, rows * n).reshape(rows, n)
    bias = kf.synth_normal(42, 1.0, n_out)
    res = kf.synth_normal(43, 1.0, rows * n_out).reshape(rows, n_out)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8_0)
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemm_i8(kf.TYPE_Q8_0, _tensor(w, cuda), act, y, rows, n, n_out, bias=_tensor(bias, cuda), res=_tensor(res, cuda))
    torch.cuda.synchronize()
    want = oracle.matmul_slice(kf.TYPE_Q8_0, w, n, n_out, x, bias) + res
    _close(y.cpu().numpy(), want)


Q4K_GEMM_SHAPES = [(9, 256, 64), (2, 256, 40), (17, 1024, 1000), (130, 512, 200), (256, 4096, 384), (33, 14336, 96),
                   (129, 2304, 130)]


@pytest.mark.parametrize("rows,n,n_out", Q4K_GEMM_SHAPES)
def test_gemm_q4_k_matches_cpu_backend(cuda, rows, n, n_out):
    """The q4_K int8 MFMA GEMM against matmul_slice, with bias and residual; ragged tiles and nine-super-block rows."""
    import torch

    w = _weights(kf.TYPE_Q4_K, n_out, n, seed=50 + rows)
    x = kf.synth_normal(51 + rows, 1.0, rows * n).reshape(rows, n)
    bias = kf.synth_normal(52, 1.0, n_out)
    res = kf.synth_normal(53, 1.0, rows * n_out).reshape(rows, n_out)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8K)
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemm_i8(kf.TYPE_Q4_K, _tensor(w, cuda), act, y, rows, n, n_out, bias=_tensor(bias, cuda), res=_tensor(res, cuda))
    torch.cuda.synchronize()
    _close(y.cpu().numpy(), oracle.matmul_slice(kf.TYPE_Q4_K, w, n, n_out, x, bias) + res)


def test_gemm_q4_k_random_blocks_and_extreme_sums(cuda):
    """Random header bytes (6-bit scales and mins up to 63) and activation blocks at full scale, so the group sums
    reach +-4064 and the exact mins product (64 hi + lo split) is exercised at its limits."""
    import torch

    rng = np.random.default_rng(7)
    rows, n, n_out = 70, 1024, 136
    w = _random_blocks(kf.TYPE_Q4_K, n_out, n, rng)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    # Q8K rounds the super-block's first max-|v| value to -127 and clamps the opposite sign at +127, so a group at the
    # maximum and one at minus the maximum give sums of -4064 and +4064
    x[3, :32] = 4.0
    x[3, 32:64] = -4.0
    x[5, 256:288] = -4.0
    x[5, 288:320] = 4.0
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8K)
    _, _, _, _, s32 = kf.act_views(act, rows, n)
    sums = s32.cpu().numpy()
    assert sums.max() == 4064 and sums.min() == -4064
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemm_i8(kf.TYPE_Q4_K, _tensor(w, cuda), act, y, rows, n, n_out)
    torch.cuda.synchronize()
    _close(y.cpu().numpy(), oracle.matmul_slice(kf.TYPE_Q4_K, w, n, n_out, x))


# Rows of the full-size prefill checks: every 97th row, the rows either side of the 64- and 128-row tile edges at both
# ends, and the last rows (whole rows, so every column tile, the tail-split ones included)
PREFILL_ROWS = sorted(set(range(0, 2048, 97)) | {63, 64, 127, 128, 1919, 1920, 1983, 1984, 2046, 2047})


@pytest.mark.parametrize("n,n_out", [(4096, 14336), (14336, 4096)])
def test_gemm_q4_k_prefill_shapes_match_gemv(cuda, n, n_out):
    """Q4_K at the Llama-3-8B shapes and M = 2048: the PREFILL_ROWS rows of the GEMM against the GEMV of that row on
    the same quantized activations, and against the CPU backend's matmul_slice (rows are independent)."""
    import torch

    rows = 2048
    w = _tensor(_weights(kf.TYPE_Q4_K, n_out, n, seed=3), cuda)
    x = _tensor(kf.synth_normal(4, 1.0, rows * n).reshape(rows, n), cuda)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(x, act, kf.ACT_Q8K)
    y = torch.empty((rows, n_out), device=cuda)
    kf.gemm_i8(kf.TYPE_Q4_K, w, act, y, rows, n, n_out)
    views = kf.act_views(act, rows, n)
    one = kf.alloc_act(1, n, cuda)
    oviews = kf.act_views(one, 1, n)
    yr = torch.empty((1, n_out), device=cuda)
    for r in PREFILL_ROWS:
        for src, dst in zip(views, oviews):
            dst.copy_(src[r : r + 1])
        kf.gemv(kf.TYPE_Q4_K, w, one, yr, 1, n, n_out)
        torch.cuda.synchronize()
        _close(y[r : r + 1].cpu().numpy(), yr.cpu().numpy())
    # rows are independent: the sampled rows against the CPU backend itself
    sample = PREFILL_ROWS
    want = oracle.matmul_slice(kf.TYPE_Q4_K, w.cpu().numpy(), n, n_out, x[sample].cpu().numpy())
    _close(y[sample].cpu().numpy(), want)


@pytest.mark.parametrize("rows,n_out", [(9, 96), (40, 96), (40, 12300), (200, 96)])
def test_matmul_q4_k_many_rows(cuda, rows, n_out):
    """kf_hip_matmul with many q4_K rows (the multi-row product below the GEMM crossover, the tile GEMM above it:
    200 rows, or 40 rows over 97 column tiles); results as the CPU backend's."""
    import torch

    n = 512
    w = _weights(kf.TYPE_Q4_K, n_out, n, seed=60 + rows)
    x = kf.synth_normal(61 + rows, 1.0, rows * n).reshape(rows, n)
    act = kf.alloc_act(rows, n, cuda)
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.matmul(kf.TYPE_Q4_K, _tensor(w, cuda), _tensor(x, cuda), act, y, n_out)
    torch.cuda.synchronize()
    _close(y.cpu().numpy(), oracle.matmul_slice(kf.TYPE_Q4_K, w, n, n_out, x))


@pytest.mark.parametrize("n,n_out", [(4096, 14336), (14336, 4096)])
def test_gemm_prefill_shapes_match_gemv(cuda, n, n_out):
    """Config C4 at full size (M = 2048): the PREFILL_ROWS rows of the GEMM against the GEMV of that row on the same
    quantized activations, and against the CPU backend's matmul_slice (rows are independent)."""
    import torch

    rows = 2048
    w = _tensor(_weights(kf.TYPE_Q8_0, n_out, n, seed=0), cuda)
    x = _tensor(kf.synth_normal(1, 1.0, rows * n).reshape(rows, n), cuda)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(x, act, kf.ACT_Q8_0)
    y = torch.empty((rows, n_out), device=cuda)
    kf.gemm_i8(kf.TYPE_Q8_0, w, act, y, rows, n, n_out)
    q, d16, s16, d32, s32 = kf.act_views(act, rows, n)
    one = kf.alloc_act(1, n, cuda)
    oq, od16, os16, od32, os32 = kf.act_views(one, 1, n)
    yr = torch.empty((1, n_out), device=cuda)
    for r in PREFILL_ROWS:
        for src, dst in ((q, oq), (d16, od16), (s16, os16), (d32, od32), (s32, os32)):
            dst.copy_(src[r : r + 1])
        kf.gemv(kf.TYPE_Q8_0, w, one, yr, 1, n, n_out)
        torch.cuda.synchronize()
        _close(y[r : r + 1].cpu().numpy(), yr.cpu().numpy())
    # rows are independent: the sampled rows against the CPU backend itself
    sample = PREFILL_ROWS
    want = oracle.matmul_slice(kf.TYPE_Q8_0, w.cpu().numpy(), n, n_out, x[sample].cpu().numpy())
    _close(y[sample].cpu().numpy(), want)


@pytest.mark.parametrize("ty", [kf.TYPE_Q8_0, kf.TYPE_Q4_K])
@pytest.mark.parametrize("rows", [1, 2, 5, 8, 9, 13, 16, 23, 32, 33, 40])
def test_matmul_reference_row_counts(cuda, ty, rows):
    """kf_hip_matmul at the row counts of the reference's differential test (crates/kf-backend-cuda/tests/quant.rs:46-64),
    200 output rows (off the 16-row groups): whichever product the row count selects matches the CPU backend."""
    n, n_out = 1024, 200
    w = _weights(ty, n_out, n, 70 + rows)
    x = kf.synth_normal(71 + rows, 1.0, rows * n).reshape(rows, n)
    act = kf.alloc_act(rows, n, cuda)
    import torch

    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.matmul(ty, _tensor(w, cuda), _tensor(x, cuda), act, y, n_out)
    torch.cuda.synchronize()
    _close(y.cpu().numpy(), oracle.matmul_slice(ty, w, n, n_out, x))


@pytest.mark.parametrize("n_out", [4104, 8232, 16400])
def test_matmul_q4_k_few_rows_tiles_per_block(cuda, n_out):
    """q4_K few-row product of one matrix with two, four and eight 16-row tiles a block (the tile count follows the
    number of tiles against the CU count; ragged last tile) against the CPU backend's matmul_slice."""
    import torch

    ty, n, rows = kf.TYPE_Q4_K, 1024, 8
    w = _weights(ty, n_out, n, n_out)
    x = kf.synth_normal(n_out + 1, 1.0, rows * n).reshape(rows, n)
    act = kf.alloc_act(rows, n, cuda)
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.matmul(ty, _tensor(w, cuda), _tensor(x, cuda), act, y, n_out)
    torch.cuda.synchronize()
    _close(y.cpu().numpy(), oracle.matmul_slice(ty, w, n, n_out, x))


@pytest.mark.parametrize("rows", [96, 128, 192, 256])
def test_matmul_q4_k_cost_model_rows(cuda, rows):
    """kf_hip_matmul on q4_K between the few-row product and the tile GEMM (the cost model picks either, ragged
    n_out) against the CPU backend's matmul_slice."""
    import torch

    ty, n, n_out = kf.TYPE_Q4_K, 1024, 200
    w = _weights(ty, n_out, n, 90 + rows)
    x = kf.synth_normal(91 + rows, 1.0, rows * n).reshape(rows, n)
    act = kf.alloc_act(rows, n, cuda)
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.matmul(ty, _tensor(w, cuda), _tensor(x, cuda), act, y, n_out)
    torch.cuda.synchronize()
    _close(y.cpu().numpy(), oracle.matmul_slice(ty, w, n, n_out, x))


@pytest.mark.parametrize("rows", [96, 256])
def test_matmul_q4_k_wide_k_few_row_and_gemm(cuda, rows):
    """Wide K (down's 14336 columns, a small n_out): the cost model keeps the few-row product here (its weight pass
    is cheap against a GEMM round of 56 super-blocks), which then carries 96 or 256 rows in 64-row passes. The
    selected kf_hip_matmul must equal that product (kf_hip_gemv) bit for bit; the few-row product and the tile GEMM
    (kf_hip_gemm_i8) each against the CPU backend's int8 path on every 7th row."""
    import torch

    ty, n, n_out = kf.TYPE_Q4_K, 14336, 40
    w = _weights(ty, n_out, n, 95 + rows)
    x = kf.synth_normal(96 + rows, 1.0, rows * n).reshape(rows, n)
    wt, xt = _tensor(w, cuda), _tensor(x, cuda)
    act = kf.alloc_act(rows, n, cuda)
    outs = {}
    for name in ("matmul", "gemv", "gemm"):
        y = torch.full((rows, n_out), float("nan"), device=cuda)
        if name == "matmul":
            kf.matmul(ty, wt, xt, act, y, n_out)
        elif name == "gemv":
            kf.gemv(ty, wt, act, y, rows, n, n_out)
        else:
            kf.gemm_i8(ty, wt, act, y, rows, n, n_out)
        torch.cuda.synchronize()
        outs[name] = y.cpu().numpy()
    assert np.array_equal(outs["matmul"].view(np.uint32), outs["gemv"].view(np.uint32))
    sample = np.arange(0, rows, 7)
    want = oracle.matmul_i8(ty, w, n, n_out, x[sample])
    _close(outs["gemv"][sample], want)
    _close(outs["gemm"][sample], want)


LLAMA_SHAPES = {"qkv": (4096, 6144), "o": (4096, 4096), "gate": (4096, 14336), "down": (14336, 4096)}


@pytest.mark.parametrize("shape", list(LLAMA_SHAPES))
@pytest.mark.parametrize("rows", [8, 16, 32, 64])
def test_matmul_q8_0_small_batch_llama_shapes(cuda, shape, rows):
    """Config C3: kf_hip_matmul on Q8_0 weights at the Llama-3-8B shapes and 8 / 16 / 32 / 64 activation rows (the
    small-batch product), every 7th output column against the CPU backend's matmul_slice on those weight rows (output
    columns are independent) (crates/kf-backend-cuda/tests/quant.rs:46-112)."""
    import torch

    n, n_out = LLAMA_SHAPES[shape]
    w = _weights(kf.TYPE_Q8_0, n_out, n, seed=200 + n_out)
    x = kf.synth_normal(201 + rows, 1.0, rows * n).reshape(rows, n)
    act = kf.alloc_act(rows, n, cuda)
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.matmul(kf.TYPE_Q8_0, _tensor(w, cuda), _tensor(x, cuda), act, y, n_out)
    torch.cuda.synchronize()
    cols = np.arange(0, n_out, 7)
    want = oracle.matmul_slice(kf.TYPE_Q8_0, np.ascontiguousarray(w[cols]), n, len(cols), x)
    got = y.cpu().numpy()
    assert np.isfinite(got).all()
    _close(got[:, cols], want)


@pytest.mark.parametrize("variant", ["11", "14"])
@pytest.mark.parametrize("rows,n,n_out", [(49, 256, 40), (53, 4096, 300), (64, 1280, 520), (57, 14336, 96), (64, 768, 4100)])
def test_gemm_q8_0_all_rows_one_pass_variants(cuda, knobs, variant, rows, n, n_out):
    """49..64 Q8_0 rows in one weight pass (activation rows staged in LDS per K chunk), both (waves) variants: ragged
    row counts, a single chunk, K split over waves with a chunk count that is not a multiple of the waves, a last
    weight tile past n_out, against the CPU backend."""
    import torch

    knobs.setenv("KF_GEMM_MR", variant)
    knobs.setenv("KF_GEMM_SK", "0")  # the split-K form takes these rows first
    rng = np.random.default_rng(rows * 7 + n_out)
    w = _weights(kf.TYPE_Q8_0, n_out, n, seed=rows + n)
    x = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    bias = kf.synth_normal(5, 1.0, n_out)
    res = kf.synth_normal(6, 1.0, rows * n_out).reshape(rows, n_out)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8_0)
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemm_i8(kf.TYPE_Q8_0, _tensor(w, cuda), act, y, rows, n, n_out, bias=_tensor(bias, cuda), res=_tensor(res, cuda))
    torch.cuda.synchronize()
    _close(y.cpu().numpy(), oracle.matmul_slice(kf.TYPE_Q8_0, w, n, n_out, x, bias) + res)


@pytest.mark.parametrize("rows,n,n_out,splits,var", [(17, 4096, 4096, None, None), (32, 4096, 300, None, None),
                                                     (33, 14336, 4100, None, None), (33, 14336, 4100, 7, None),
                                                     (64, 4096, 14336, None, None), (50, 384, 200, None, None),
                                                     (64, 1024, 64, None, None), (24, 1024, 256, 4, None),
                                                     (40, 4096, 1000, None, 43), (64, 14336, 520, 5, 43),
                                                     (20, 4096, 700, None, 83), (64, 2048, 300, None, 162),
                                                     (1, 4096, 6144, None, None), (8, 4096, 14336, None, None),
                                                     (16, 14336, 4096, None, None), (5, 1024, 200, 3, None),
                                                     (13, 4096, 520, None, 162)])
def test_gemm_q8_0_split_k(cuda, knobs, rows, n, n_out, splits, var):
    """1..64 Q8_0 rows with K split across blocks (partials summed in split order by the last block of each tile),
    forced on for every size (KF_GEMM_SK=1; by default it takes matrices above 4096 x 4096): ragged rows and output
    tiles (one to sixteen rows in one staged 16-row tile), split counts that do not divide the chunks (7 of 56; 4 of
    4: one chunk a split), the chunk forms (4, 8, 16 groups; two or three stages: KF_GEMM_SK_V), three calls in a row
    on one stream (the tickets return to zero), bias and residual; against the CPU backend, bit-identical between
    calls (deterministic), and within the f32 bar of the scratch-free products (KF_GEMM_SK=0)."""
    import torch

    knobs.setenv("KF_GEMM_SK", "1")
    if splits:
        knobs.setenv("KF_GEMM_SK_S", str(splits))
    if var:
        knobs.setenv("KF_GEMM_SK_V", str(var))

    rng = np.random.default_rng(rows * 13 + n + n_out)
    w = _weights(kf.TYPE_Q8_0, n_out, n, seed=rows + n_out)
    x = (rng.standard_normal((rows, n)) * 2).astype(np.float32)
    bias = kf.synth_normal(7, 1.0, n_out)
    res = kf.synth_normal(8, 1.0, rows * n_out).reshape(rows, n_out)
    wt, bt, rt = _tensor(w, cuda), _tensor(bias, cuda), _tensor(res, cuda)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8_0)
    outs = []
    for _ in range(3):
        y = torch.full((rows, n_out), float("nan"), device=cuda)
        kf.gemm_i8(kf.TYPE_Q8_0, wt, act, y, rows, n, n_out, bias=bt, res=rt)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    want = oracle.matmul_slice(kf.TYPE_Q8_0, w, n, n_out, x, bias) + res
    _close(outs[0], want)
    knobs.setenv("KF_GEMM_SK", "0")
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemm_i8(kf.TYPE_Q8_0, wt, act, y, rows, n, n_out, bias=bt, res=rt)
    torch.cuda.synchronize()
    _close(outs[0], y.cpu().numpy())


@pytest.mark.parametrize("kq", ["0", "1"])
@pytest.mark.parametrize("rows,n,n_out", [(2048, 4096, 14336), (130, 2048, 600), (257, 1024, 300), (96, 14336, 512)])
def test_gemm_q4_k_tail_halves(cuda, knobs, rows, n, n_out, kq):
    """The q4_K GEMMs' tail split, both kernels (KF_Q4K_KQ: 0 the split-scale kernel, two K halves; 1 the
    one-MFMA-per-group kernel, 2-4 K ranges): tiles of a last round at most half full (all of them when the grid is
    below half the CUs) run over K ranges whose partial tiles the last to arrive adds in order. Against the unsplit
    kernel (KF_GEMM_NO_TAIL) within the f32 bar, bit-identical over two calls on one stream (the tickets return to
    zero), and the smaller shapes against the CPU backend; 4, 8 and 56 super-blocks a row, ragged tiles."""
    import torch

    knobs.setenv("KF_Q4K_KQ", kq)

    w = _weights(kf.TYPE_Q4_K, n_out, n, seed=rows + n)
    x = kf.synth_normal(rows + 3, 1.0, rows * n).reshape(rows, n)
    bias = kf.synth_normal(5, 1.0, n_out)
    wt, bt = _tensor(w, cuda), _tensor(bias, cuda)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8K)
    outs = []
    for _ in range(2):
        y = torch.full((rows, n_out), float("nan"), device=cuda)
        kf.gemm_i8(kf.TYPE_Q4_K, wt, act, y, rows, n, n_out, bias=bt)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    knobs.setenv("KF_GEMM_NO_TAIL", "1")
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemm_i8(kf.TYPE_Q4_K, wt, act, y, rows, n, n_out, bias=bt)
    torch.cuda.synchronize()
    _close(outs[0], y.cpu().numpy())
    if rows * n_out <= 300 * 600:
        _close(outs[0], oracle.matmul_slice(kf.TYPE_Q4_K, w, n, n_out, x, bias))


@pytest.mark.parametrize("rows,n,n_out", [(2048, 4096, 14336), (300, 1024, 1000), (129, 14336, 600)])
def test_gemm_q8_0_tail_halves(cuda, knobs, rows, n, n_out):
    """The q8_0 tile GEMM's tail split (two blocks a CU: a last round at most half full, or a grid below half of
    them, runs its tiles as two K halves added in half order by the second to arrive): against the unsplit kernel
    (KF_GEMM_NO_TAIL) within the f32 bar, bit-identical over two calls, the smaller shapes against the CPU backend."""
    import torch

    w = _weights(kf.TYPE_Q8_0, n_out, n, seed=rows + n)
    x = kf.synth_normal(rows + 7, 1.0, rows * n).reshape(rows, n)
    bias = kf.synth_normal(6, 1.0, n_out)
    wt, bt = _tensor(w, cuda), _tensor(bias, cuda)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8_0)
    outs = []
    for _ in range(2):
        y = torch.full((rows, n_out), float("nan"), device=cuda)
        kf.gemm_i8(kf.TYPE_Q8_0, wt, act, y, rows, n, n_out, bias=bt)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    knobs.setenv("KF_GEMM_NO_TAIL", "1")
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemm_i8(kf.TYPE_Q8_0, wt, act, y, rows, n, n_out, bias=bt)
    torch.cuda.synchronize()
    _close(outs[0], y.cpu().numpy())
    if rows * n_out <= 300 * 1000:
        _close(outs[0], oracle.matmul_slice(kf.TYPE_Q8_0, w, n, n_out, x, bias))


@pytest.mark.parametrize("rows,n,n_out", [(96, 14336, 600), (130, 4096, 4096), (250, 14336, 520), (65, 4096, 6144)])
def test_gemm_q8_0_row_slices(cuda, knobs, rows, n, n_out):
    """65.. q8_0 rows as 64-row slices through the small-batch products (the cost model's pick at down- and O-like
    shapes up to a few hundred rows; KF_GEMM_SLICE forces each form): ragged last slices (2, 58 and 1 rows), bias and
    residual; the sliced and tile forms within the f32 bar of each other, and the auto choice against the CPU backend."""
    import torch

    w = _weights(kf.TYPE_Q8_0, n_out, n, seed=rows + 11)
    x = kf.synth_normal(rows + 13, 1.0, rows * n).reshape(rows, n)
    bias = kf.synth_normal(9, 1.0, n_out)
    res = kf.synth_normal(10, 1.0, rows * n_out).reshape(rows, n_out)
    wt, bt, rt = _tensor(w, cuda), _tensor(bias, cuda), _tensor(res, cuda)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8_0)
    outs = {}
    for force in (None, "1", "0"):
        if force is None:
            knobs.delenv("KF_GEMM_SLICE", raising=False)
        else:
            knobs.setenv("KF_GEMM_SLICE", force)
        y = torch.full((rows, n_out), float("nan"), device=cuda)
        kf.gemm_i8(kf.TYPE_Q8_0, wt, act, y, rows, n, n_out, bias=bt, res=rt)
        torch.cuda.synchronize()
        outs[force] = y.cpu().numpy()
    _close(outs["1"], outs["0"])
    if rows * n_out <= 250 * 600:
        _close(outs[None], oracle.matmul_slice(kf.TYPE_Q8_0, w, n, n_out, x, bias) + res)
    else:
        sample = np.arange(0, rows, 7)
        _close(outs[None][sample], oracle.matmul_slice(kf.TYPE_Q8_0, w, n, n_out, x[sample], bias) + res[sample])


def test_stream_read_probe(cuda):
    """The benchmark's read probe (kf_hip_stream_read) on ragged sizes: it runs for every per-thread count, leaves the
    sink alone (no data matches its key) and does not touch the buffer."""
    import torch

    sink = torch.zeros(1, dtype=torch.int32, device=cuda)
    for nbytes in (16, 4096 + 48, 3 << 20):
        buf = torch.arange(nbytes, dtype=torch.int64, device=cuda).to(torch.uint8)
        before = buf.clone()
        for p in (4, 8, 16):
            kf.stream_read(buf, sink, p)
        torch.cuda.synchronize()
        assert torch.equal(buf, before)
    assert int(sink.item()) == 0
