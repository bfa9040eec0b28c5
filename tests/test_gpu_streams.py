"""Ownership of the split-K scratch across streams and graphs, through the C ABI: two streams running split products at
once each keep their own slot (every output bit-identical to the one-stream result); a third stream takes the
scratch-free kernels (bit-identical to KF_GEMM_NO_TAIL); kf_hip_release_stream hands a slot to the next stream; a
captured product uses the graph slot, so a graph replayed on another stream beside direct calls gives the split result
on every replay, as the direct calls do; with KF_CAPTURE_NO_SPLIT the graph records the scratch-free kernels."""
import numpy as np
import pytest

import kungfu_amd as kf

pytestmark = pytest.mark.gpu

ROWS, N, N_OUT = 256, 4096, 4096  # 32 q4_K tiles: under half the CUs, so every tile runs as K halves


def _tensor(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _bits(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.fixture(scope="module")
def case(cuda):
    w = kf.quantize(kf.TYPE_Q4_K, kf.synth_normal(101, 0.02, N * N_OUT).reshape(N_OUT, N))
    x = kf.synth_normal(102, 1.0, ROWS * N).reshape(ROWS, N)
    act = kf.alloc_act(ROWS, N, cuda)
    kf.quant_act(_tensor(x, cuda), act, kf.ACT_Q8K)
    return _tensor(w, cuda), act


def _run(cuda, case, stream=None, y=None):
    """One product into y (a new NaN-filled output when None, made ready before a launch on another stream)."""
    import torch

    wt, act = case
    if y is None:
        y = torch.full((ROWS, N_OUT), float("nan"), device=cuda)
        torch.cuda.synchronize()
    kf.gemm_i8(kf.TYPE_Q4_K, wt, act, y, ROWS, N, N_OUT, stream=stream)
    return y


def _refs(cuda, case, knobs):
    import torch

    split = _run(cuda, case)  # the default stream holds a slot from the earlier products (or takes one now)
    knobs.setenv("KF_GEMM_NO_TAIL", "1")
    plain = _run(cuda, case)
    knobs.delenv("KF_GEMM_NO_TAIL")
    torch.cuda.synchronize()
    return _bits(split), _bits(plain)


def test_two_streams_keep_their_own_slots_and_a_third_runs_without(cuda, case, knobs):
    import torch

    split, plain = _refs(cuda, case, knobs)
    b, c = torch.cuda.Stream(), torch.cuda.Stream()
    try:
        # the default stream and b at once, several products each: tickets and partials never shared
        ys_a = [torch.full((ROWS, N_OUT), float("nan"), device=cuda) for _ in range(4)]
        ys_b = [torch.full((ROWS, N_OUT), float("nan"), device=cuda) for _ in range(4)]
        torch.cuda.synchronize()
        for ya, yb in zip(ys_a, ys_b):
            _run(cuda, case, y=ya)
            _run(cuda, case, stream=b.cuda_stream, y=yb)
        torch.cuda.synchronize()
        for y in ys_a + ys_b:
            assert np.array_equal(_bits(y), split)
        # both slots held: c takes the scratch-free kernel
        y = _run(cuda, case, stream=c.cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(y), plain)
        # b's slot released: c gets it and splits
        kf.release_stream(b.cuda_stream)
        y = _run(cuda, case, stream=c.cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(y), split)
    finally:
        kf.release_stream(b.cuda_stream)
        kf.release_stream(c.cuda_stream)


def test_q8_0_split_k_on_two_streams_at_once(cuda, knobs):
    import torch

    rows, n, n_out = 32, 4096, 14336
    knobs.setenv("KF_GEMM_SK", "1")
    w = _tensor(kf.quantize(kf.TYPE_Q8_0, kf.synth_normal(103, 0.02, n * n_out).reshape(n_out, n)), cuda)
    act = kf.alloc_act(rows, n, cuda)
    kf.quant_act(_tensor(kf.synth_normal(104, 1.0, rows * n).reshape(rows, n), cuda), act, kf.ACT_Q8_0)

    def run(y, stream=None):
        kf.gemm_i8(kf.TYPE_Q8_0, w, act, y, rows, n, n_out, stream=stream)
        return y

    ys = [torch.full((rows, n_out), float("nan"), device=cuda) for _ in range(9)]
    torch.cuda.synchronize()
    ref = run(ys[8])
    torch.cuda.synchronize()
    ref = _bits(ref)
    b = torch.cuda.Stream()
    try:
        for i in range(4):
            run(ys[2 * i])
            run(ys[2 * i + 1], b.cuda_stream)
        torch.cuda.synchronize()
        for y in ys[:8]:
            assert np.array_equal(_bits(y), ref)
    finally:
        kf.release_stream(b.cuda_stream)


def _replays(cuda, case, g, y_graph, n=5):
    """Replays of g on stream d, each beside a direct product on the default stream, with eager work and
    synchronisation between replays; yields (replay bits, direct bits)."""
    import torch

    d = torch.cuda.Stream()
    y_direct_buf = torch.empty((ROWS, N_OUT), device=cuda)
    try:
        for i in range(n):
            y_graph.fill_(float("nan"))
            y_direct_buf.fill_(float("nan"))
            torch.cuda.synchronize()
            d.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(d):
                g.replay()
            y_direct = _run(cuda, case, y=y_direct_buf)
            torch.cuda.synchronize()
            yield i, _bits(y_graph), _bits(y_direct)
    finally:
        kf.release_stream(d.cuda_stream)


def _capture(cuda, case):
    import torch

    wt, act = case
    y_graph = torch.full((ROWS, N_OUT), float("nan"), device=cuda)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        kf.gemm_i8(kf.TYPE_Q4_K, wt, act, y_graph, ROWS, N, N_OUT)
    return g, y_graph


def test_graph_replayed_on_another_stream_beside_direct_calls(cuda, case, knobs):
    """Captured, the product takes the graph slot (the split kernel is recorded); five replays on stream d, each
    beside a direct product on the default stream (its stream slot): both give the split result every time."""
    split, plain = _refs(cuda, case, knobs)
    g, y_graph = _capture(cuda, case)
    for i, yg, yd in _replays(cuda, case, g, y_graph):
        assert np.array_equal(yg, split), f"replay {i}"
        assert np.array_equal(yd, split), f"direct call {i}"


def test_graph_capture_without_split(cuda, case, knobs):
    """KF_CAPTURE_NO_SPLIT: the graph records the scratch-free kernel (the KF_GEMM_NO_TAIL result on every replay)."""
    split, plain = _refs(cuda, case, knobs)
    knobs.setenv("KF_CAPTURE_NO_SPLIT", "1")
    g, y_graph = _capture(cuda, case)
    knobs.delenv("KF_CAPTURE_NO_SPLIT")
    for i, yg, yd in _replays(cuda, case, g, y_graph, n=3):
        assert np.array_equal(yg, plain), f"replay {i}"
        assert np.array_equal(yd, split), f"direct call {i}"
