"""Grouped products (kf_hip_gemv_group / kf_hip_matmul_group) on the GPU.

A group is the reference's segment-table product (crates/kf-backend-cuda/src/kernels/quant.cuh:301-305,447-464;
built by matmul_group_launch, crates/kf-backend-cuda/src/exec.rs:1283-1346): several weights of one type and width
stacked along their output rows against one quantized input. Every member's output must equal the member's own
kf_hip_matmul bit for bit (the same per-row arithmetic, whichever launch covers it) and the CPU backend's
matmul_slice within the parity tolerance.
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


def _close(got, want):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bad = err > ATOL + RTOL * np.abs(want)
    assert not bad.any(), f"{bad.sum()} outputs off, worst {err.max():.3e}"


def _members(ty, n, sizes, rows, dev, seed, with_bias=(), with_res=()):
    import torch

    out = []
    for k, n_out in enumerate(sizes):
        wh = kf.quantize(ty, kf.synth_normal(seed + k, 0.02, n_out * n).reshape(n_out, n))
        bias = kf.synth_normal(seed + 50 + k, 0.1, n_out).astype(np.float32) if k in with_bias else None
        res = kf.synth_normal(seed + 80 + k, 0.1, rows * n_out).reshape(rows, n_out).astype(np.float32) if k in with_res else None
        out.append(dict(wh=wh, w=_tensor(wh, dev), n_out=n_out, bias_h=bias, res_h=res,
                        bias=None if bias is None else _tensor(bias, dev), res=None if res is None else _tensor(res, dev),
                        y=torch.full((rows, n_out), float("nan"), device=dev)))
    return out


def _check(ty, ms, x, n, dev):
    import torch

    rows = x.shape[0]
    torch.cuda.synchronize()
    act = kf.alloc_act(rows, n, dev)
    for m in ms:
        y1 = torch.empty((rows, m["n_out"]), device=dev)
        kf.matmul(ty, m["w"], _tensor(x, dev), act, y1, m["n_out"], bias=m["bias"], res=m["res"])
        torch.cuda.synchronize()
        got = m["y"].cpu().numpy()
        assert np.array_equal(got, y1.cpu().numpy()), f"member of {m['n_out']} rows differs from its own product"
        want = oracle.matmul_slice(ty, m["wh"], n, m["n_out"], x, m["bias_h"])
        if m["res_h"] is not None:
            want = want + m["res_h"]
        _close(got, want)


@pytest.mark.parametrize("ty,n,sizes", [
    (kf.TYPE_Q4_K, 4096, (512, 128, 128)),       # Q/K/V at a reduced head count
    (kf.TYPE_Q8_0, 4096, (256, 256)),            # gate and up stored apart
    (kf.TYPE_Q4_K, 14336, (96, 40)),             # several waves a row
    (kf.TYPE_Q8_0, 128, (7, 33, 100, 1)),        # four ragged members: boundaries inside a block's rows
])
def test_group_one_row_single_launch(cuda, ty, n, sizes):
    import torch

    ms = _members(ty, n, sizes, 1, cuda, seed=11, with_bias=(0,), with_res=(len(sizes) - 1,))
    x = kf.synth_normal(3, 1.0, n).reshape(1, n)
    act = kf.alloc_act(1, n, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.act_kind(ty))
    kf.gemv_group(ty, [(m["w"], m["y"], m["bias"], m["res"]) for m in ms], act, 1, n)
    torch.cuda.synchronize()
    _check(ty, ms, x, n, cuda)


@pytest.mark.parametrize("ty,rows,n,sizes", [
    (kf.TYPE_Q4_K, 1, 1024, (64, 96, 32)),       # one row: one launch that quantizes x itself
    (kf.TYPE_Q8_0, 1, 4096, (256, 256)),
    (kf.TYPE_Q4_K, 1, 14336, (96, 40)),
    (kf.TYPE_Q4_K, 3, 1024, (64, 96)),           # the multi-row product per member
    (kf.TYPE_Q8_0, 64, 4096, (256, 128)),        # the int8 GEMM per member
    (kf.TYPE_Q4_K, 200, 1024, (256, 128)),       # the q4_K GEMM per member
    (kf.TYPE_Q6_K, 1, 512, (64, 32)),            # q6_K: each member's own product
    (kf.TYPE_Q5_K, 2, 512, (48, 16)),
])
def test_matmul_group(cuda, ty, rows, n, sizes):
    import torch

    ms = _members(ty, n, sizes, rows, cuda, seed=rows + n, with_bias=(1,), with_res=(0,))
    x = (kf.synth_normal(rows * 7 + 1, 1.0, rows * n).reshape(rows, n)).astype(np.float32)
    act = kf.alloc_act(rows, n, cuda)
    kf.matmul_group(ty, [(m["w"], m["y"], m["bias"], m["res"]) for m in ms], _tensor(x, cuda), act)
    torch.cuda.synchronize()
    _check(ty, ms, x, n, cuda)


def test_group_members_in_one_output_buffer(cuda):
    """Members writing disjoint column ranges of one buffer (the stacked [n_q + n_k + n_v] layout, one row)."""
    import torch

    ty, n, sizes = kf.TYPE_Q4_K, 2048, (256, 64, 64)
    ms = _members(ty, n, sizes, 1, cuda, seed=5)
    yall = torch.full((1, sum(sizes)), float("nan"), device=cuda)
    at = 0
    for m in ms:
        m["y"] = yall[:, at : at + m["n_out"]]
        at += m["n_out"]
    x = kf.synth_normal(9, 1.0, n).reshape(1, n)
    act = kf.alloc_act(1, n, cuda)
    kf.matmul_group(ty, [(m["w"], m["y"], None, None) for m in ms], _tensor(x, cuda), act)
    torch.cuda.synchronize()
    assert not torch.isnan(yall).any()
    _check(ty, ms, x, n, cuda)
