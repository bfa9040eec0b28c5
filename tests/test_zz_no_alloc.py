"""kf_hip_matmul_noalloc (the entry point that allocates nothing: its activation scratch is a static per-GPU array in the
library) against kf_hip_matmul with a caller-allocated scratch, through the C ABI: bit-identical outputs on two calls in
a row, the second smaller than the first (the array keeps the first call's contents), and both within the north-star
bar of the CPU backend's matmul_slice (crates/kf-backend-cpu/src/ops.rs:304-346)."""
import numpy as np
import pytest

import kungfu_amd as kf
import oracle

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4


def _t(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("ty", [kf.TYPE_Q8_0, kf.TYPE_Q4_K])
def test_noalloc_matches_matmul_twice_shrinking(cuda, ty):
    import torch

    n = 4096
    cases = [(256, 640, 11), (3, 200, 12)]  # (rows, n_out, seed): the second call is smaller
    for rows, n_out, seed in cases:
        print(f"noalloc case ty={ty} rows={rows} n={n} n_out={n_out}", flush=True)
        w = kf.quantize(ty, kf.synth_normal(seed, 0.02, n_out * n).reshape(n_out, n))
        x = kf.synth_normal(seed + 100, 1.0, rows * n).reshape(rows, n)
        bias = kf.synth_normal(seed + 200, 1.0, n_out)
        w_, x_, b_ = _t(w, cuda), _t(x, cuda), _t(bias, cuda)
        y_ref = torch.full((rows, n_out), float("nan"), device=cuda)
        act = kf.alloc_act(rows, n, cuda)
        kf.matmul(ty, w_, x_, act, y_ref, n_out, bias=b_)
        y = torch.full((rows, n_out), float("nan"), device=cuda)
        kf.matmul_noalloc(ty, w_, x_, y, n_out, bias=b_)
        torch.cuda.synchronize()
        got, ref = y.cpu().numpy(), y_ref.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        want = oracle.matmul_slice(ty, w, n, n_out, x, bias)
        err = np.abs(got.astype(np.float64) - want)
        assert (err <= ATOL + RTOL * np.abs(want)).all(), f"worst {err.max():.3e}"


def test_noalloc_rejects_activations_past_its_scratch(cuda):
    """A call whose activations need more than the static scratch fails on the host with a clear error (no launch)."""
    import torch

    limit = kf.lib().kf_hip_noalloc_scratch_bytes()
    n = 16384
    rows = 1
    while kf.act_bytes(rows, n) <= limit:
        rows *= 2
    x = torch.empty((rows, n), device=cuda)
    w = torch.empty(16, dtype=torch.uint8, device=cuda)
    y = torch.empty((rows, 1), device=cuda)
    with pytest.raises(kf.KfError) as e:
        kf.matmul_noalloc(kf.TYPE_Q8_0, w, x, y, 1)
    assert "no-allocation" in str(e.value)
