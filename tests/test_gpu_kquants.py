"""GPU parity of the q5_K and q6_K products through the C ABI: per-block integers bit-exact against the oracle (the
reference's dot_i8 integers), f32 outputs within |got - want| <= 1e-4 + 1e-3 |want| of the CPU backend's
matmul_slice, for one and several activation rows, ragged shapes, bias and residual."""
import numpy as np
import pytest

import kungfu_amd as kf
import oracle

pytestmark = pytest.mark.gpu


def _tensor(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _random_blocks(ty, n_out, n_in, rng):
    """Random block bytes with f16 scales in the range real weights use (2^-14..2^-7: d and dmin of q5_K, d of q6_K);
    larger ones give outputs whose terms reach hundreds, where an output that cancels to near zero sits below the f32
    rounding of its terms in any summation order."""
    size = kf.BLOCK[ty][1]
    w = rng.integers(0, 256, (n_out, n_in // 256, size), dtype=np.uint8)
    for at in ((0, 2) if ty == kf.TYPE_Q5_K else (208,)):
        bits = (((1 + rng.integers(0, 8, w.shape[:2])) << 10) | rng.integers(0, 1024, w.shape[:2])).astype(np.uint16)
        w[:, :, at : at + 2] = bits.view(np.uint8).reshape(w.shape[0], w.shape[1], 2)
    return w.reshape(n_out, -1)


def _gauss_blocks(ty, n_out, n_in, seed):
    """Blocks from the build's encoder on N(0, 0.02) weights, the scale real checkpoints have: outputs of magnitude a
    few units, where the f32 rounding of any summation order stays far below the north-star bar."""
    return kf.quantize(ty, kf.synth_normal(seed, 0.02, n_out * n_in).reshape(n_out, n_in))


def _close(got, want):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = 1e-4 + 1e-3 * np.abs(want.astype(np.float64))
    assert (err <= bound).all(), f"max err {err.max():.3e} at {np.unravel_index(np.argmax(err - bound), err.shape)}"


@pytest.mark.parametrize("ty", [kf.TYPE_Q5_K, kf.TYPE_Q6_K])
@pytest.mark.parametrize("rows,n,n_out", [(1, 256, 5), (2, 1024, 7), (3, 4096, 3)])
def test_block_ints_bit_exact(cuda, ty, rows, n, n_out):
    import torch

    rng = np.random.default_rng(n + n_out + ty)
    w = _random_blocks(ty, n_out, n, rng)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.act_kind(ty))
    per = n // 256 if ty == kf.TYPE_Q6_K else 2 * (n // 256)
    out = torch.zeros(n_out * rows * per, dtype=torch.int32, device=cuda)
    kf.block_ints(ty, _tensor(w, cuda), act, out, rows, n, n_out)
    got = out.cpu().numpy().reshape(n_out, rows, per)
    q, _, s16 = oracle.quantize_activations(kf.act_kind(ty), x)
    for o in range(n_out):
        for r in range(rows):
            assert np.array_equal(got[o, r], oracle.block_ints(ty, w[o], q[r], s16[r])), (o, r)


@pytest.mark.parametrize("ty", [kf.TYPE_Q5_K, kf.TYPE_Q6_K])
@pytest.mark.parametrize("rows,n,n_out", [(1, 256, 1), (1, 2304, 33), (1, 4096, 520), (1, 14336, 300), (3, 1024, 77),
                                          (8, 4096, 64), (13, 2048, 40)])
def test_product_matches_cpu_backend(cuda, ty, rows, n, n_out):
    """kf_hip_matmul (quant_act + the q5_K/q6_K product) against matmul_slice, with bias and residual; 13 rows take two
    launches (eight rows a weight pass), 2304 columns a ragged wave pass (nine super-blocks)."""
    import torch

    rng = np.random.default_rng(rows * 1000 + n + n_out + ty)
    w = kf.quantize(ty, kf.synth_normal(ty + n, 0.02, n * n_out).reshape(n_out, n))
    x = rng.standard_normal((rows, n)).astype(np.float32)
    bias = rng.standard_normal(n_out).astype(np.float32)
    res = rng.standard_normal((rows, n_out)).astype(np.float32)
    act = kf.alloc_act(rows, n, cuda)
    y = torch.empty((rows, n_out), device=cuda)
    kf.matmul(ty, _tensor(w, cuda), _tensor(x, cuda), act, y, n_out, bias=_tensor(bias, cuda), res=_tensor(res, cuda))
    torch.cuda.synchronize()
    want = oracle.matmul_slice(ty, w, n, n_out, x, bias) + res
    _close(y.cpu().numpy(), want)


def test_product_on_random_blocks(cuda):
    """Random block bytes (every scale and bit pattern) at one and five rows through kf_hip_gemv directly."""
    import torch

    rng = np.random.default_rng(11)
    for ty in (kf.TYPE_Q5_K, kf.TYPE_Q6_K):
        n, n_out = 1536, 29
        w = _random_blocks(ty, n_out, n, rng)
        for rows in (1, 5):
            x = rng.standard_normal((rows, n)).astype(np.float32)
            act = kf.alloc_act(rows, n, cuda)
            kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8K)
            y = torch.empty((rows, n_out), device=cuda)
            kf.gemv(ty, _tensor(w, cuda), act, y, rows, n, n_out)
            torch.cuda.synchronize()
            _close(y.cpu().numpy(), oracle.matmul_slice(ty, w, n, n_out, x))


@pytest.mark.parametrize("ty", [kf.TYPE_Q5_K, kf.TYPE_Q6_K])
@pytest.mark.parametrize("rows,n,n_out", [(2, 512, 16), (20, 4096, 1000), (17, 2304, 45), (16, 14336, 200), (33, 1024, 130)])
def test_multi_row_matrix_cores(cuda, ty, rows, n, n_out):
    """Several rows of q5_K / q6_K on the matrix cores (16 activation rows a weight pass, K split over a block's
    waves): chunks of 16 rows past the first, ragged last tiles, 14336 columns; 2304 columns (nine super-blocks a row)
    leave q6_K rows 2-byte aligned, which the per-lane product takes instead. Encoder blocks of N(0, 0.02) weights
    (every bit pattern is covered by the block-integer test), with bias and residual, against the CPU backend's int8
    path (ops::matmul_i8: the same quantized activations and dot_i8 integers) at the north-star bar."""
    import torch

    rng = np.random.default_rng(rows * 31 + n + n_out + ty)
    w = _gauss_blocks(ty, n_out, n, rows * 31 + n + n_out + ty)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    bias = rng.standard_normal(n_out).astype(np.float32)
    res = rng.standard_normal((rows, n_out)).astype(np.float32)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8K)
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemv(ty, _tensor(w, cuda), act, y, rows, n, n_out, bias=_tensor(bias, cuda), res=_tensor(res, cuda))
    torch.cuda.synchronize()
    _close(y.cpu().numpy(), oracle.matmul_i8(ty, w, n, n_out, x, bias) + res)


def _gemm_bound(got, want):
    _close(got, want)


@pytest.mark.parametrize("ty", [kf.TYPE_Q5_K, kf.TYPE_Q6_K])
@pytest.mark.parametrize("rows,n,n_out", [(1, 2048, 33), (64, 2048, 256), (70, 4096, 300), (130, 2048, 520),
                                          (200, 14336, 96), (17, 6144, 257)])
def test_gemm_tile_shapes(cuda, ty, rows, n, n_out):
    """The q5_K / q6_K prefill GEMM (64 x 256 block tiles over native super-blocks): ragged row panels and column
    tiles, one row, 14336 and 6144 columns (q6_K rows 16-byte aligned: n a multiple of 2048), encoder blocks of
    N(0, 0.02) weights, with bias and residual, against the CPU backend's int8 path (the same quantized activations and
    dot_i8 integers) at the north-star bar. Every scale, min and bit pattern is covered by the block-integer test."""
    import torch

    rng = np.random.default_rng(rows * 7 + n + n_out + ty)
    w = _gauss_blocks(ty, n_out, n, 141 + n + n_out + ty)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    bias = rng.standard_normal(n_out).astype(np.float32)
    res = rng.standard_normal((rows, n_out)).astype(np.float32)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8K)
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemm_i8(ty, _tensor(w, cuda), act, y, rows, n, n_out, bias=_tensor(bias, cuda), res=_tensor(res, cuda))
    torch.cuda.synchronize()
    _gemm_bound(y.cpu().numpy(), oracle.matmul_i8(ty, w, n, n_out, x, bias) + res)


@pytest.mark.parametrize("ty", [kf.TYPE_Q5_K, kf.TYPE_Q6_K])
@pytest.mark.parametrize("n,n_out", [(4096, 14336), (14336, 4096)])
def test_gemm_prefill_shapes(cuda, ty, n, n_out):
    """M = 2048 at the Llama-3-8B gate and down shapes with weights from the build's encoder: every 97th row against
    the CPU backend's float product (rows are independent), and the whole output against the few-row matrix-core
    product (kf_hip_gemv) within the same bar."""
    import torch

    rows = 2048
    w = kf.quantize(ty, kf.synth_normal(3, 0.02, n * n_out).reshape(n_out, n))
    x = kf.synth_normal(4, 1.0, rows * n).reshape(rows, n)
    wt = _tensor(w, cuda)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8K)
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemm_i8(ty, wt, act, y, rows, n, n_out)
    y2 = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemv(ty, wt, act, y2, rows, n, n_out)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    sample = np.arange(0, rows, 97)
    _close(got[sample], oracle.matmul_slice(ty, w, n, n_out, x[sample], None))
    _close(got, y2.cpu().numpy())


@pytest.mark.parametrize("ty", [kf.TYPE_Q5_K, kf.TYPE_Q6_K])
def test_gemm_shapes_it_declines(cuda, ty):
    """2304 columns: q6_K's 210-byte super-block rows are then not 16-byte aligned, so kf_hip_gemm_i8 refuses
    (KF_E_UNSUPPORTED) and kf_hip_matmul takes the few-row product; q5_K's 176-byte rows stay aligned and the GEMM takes
    them. Against the CPU backend's int8 path either way."""
    import torch

    n, n_out, rows = 2304, 40, 128
    rng = np.random.default_rng(ty)
    w = _gauss_blocks(ty, n_out, n, 187 + n + n_out + ty)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    act = kf.alloc_act(rows, n, cuda)
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8K)
    if ty == kf.TYPE_Q6_K:
        with pytest.raises(kf.KfError):
            kf.gemm_i8(ty, _tensor(w, cuda), act, y, rows, n, n_out)
    kf.matmul(ty, _tensor(w, cuda), _tensor(x, cuda), act, y, n_out)
    torch.cuda.synchronize()
    _gemm_bound(y.cpu().numpy(), oracle.matmul_i8(ty, w, n, n_out, x, None))


@pytest.mark.parametrize("ty", [kf.TYPE_Q5_K, kf.TYPE_Q6_K])
@pytest.mark.parametrize("rows", [63, 97, 256])
def test_matmul_picks_gemm_by_cost(cuda, ty, rows):
    """kf_hip_matmul around its few-row / tile GEMM switch at the gate shape (4096 -> 14336: the cost model moves to
    the GEMM at about 64 rows for q5_K and 32 for q6_K) gives the outputs of both products, within the bar."""
    import torch

    n, n_out = 4096, 14336
    rng = np.random.default_rng(rows + ty)
    w = _gauss_blocks(ty, n_out, n, 209 + n + n_out + ty)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    wt, xt = _tensor(w, cuda), _tensor(x, cuda)
    act = kf.alloc_act(rows, n, cuda)
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.matmul(ty, wt, xt, act, y, n_out)
    y2 = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemv(ty, wt, act, y2, rows, n, n_out)
    y3 = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemm_i8(ty, wt, act, y3, rows, n, n_out)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    _gemm_bound(got, y2.cpu().numpy())
    _gemm_bound(got, y3.cpu().numpy())


@pytest.mark.parametrize("ty", [kf.TYPE_Q5_K, kf.TYPE_Q6_K])
@pytest.mark.parametrize("rows,n,n_out", [(256, 14336, 4096), (100, 2048, 300), (64, 4096, 1000), (2048, 4096, 2304)])
def test_gemm_tail_splits(cuda, knobs, ty, rows, n, n_out):
    """The q5_K / q6_K GEMM's tail split: tiles of a last round at most half full (or a grid below half the CUs) run
    as 2 or 4 blocks over K ranges, added in split order by the last to arrive. Bit-identical over two calls, within
    the bar of the unsplit kernel (KF_GEMM_NO_TAIL), and the smaller shapes against the CPU backend's int8 path."""
    import torch

    rng = np.random.default_rng(rows + n + ty)
    w = _gauss_blocks(ty, n_out, n, 234 + n + n_out + ty)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    bias = rng.standard_normal(n_out).astype(np.float32)
    wt, bt = _tensor(w, cuda), _tensor(bias, cuda)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8K)
    outs = []
    for _ in range(2):
        y = torch.full((rows, n_out), float("nan"), device=cuda)
        kf.gemm_i8(ty, wt, act, y, rows, n, n_out, bias=bt)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    knobs.setenv("KF_GEMM_NO_TAIL", "1")
    y = torch.full((rows, n_out), float("nan"), device=cuda)
    kf.gemm_i8(ty, wt, act, y, rows, n, n_out, bias=bt)
    torch.cuda.synchronize()
    _gemm_bound(outs[0], y.cpu().numpy())
    if rows * n_out <= 100000:
        _gemm_bound(outs[0], oracle.matmul_i8(ty, w, n, n_out, x, bias))
