"""A GGUF file end to end on the GPU: tensors written to a GGUF file (q4_K, q6_K and q8_0 weights plus an f32 norm
weight), opened by the library's reader, uploaded from the mapped bytes through kf_hip_backend_add_weight (the
reference's WeightSource path) and multiplied; the result against the CPU backend's product on the same bytes (the
reference's real-tensor differential test, crates/kf-backend-cuda/tests/quant.rs:136-171, on a synthetic file since no
model file exists here)."""
import numpy as np
import pytest

import kungfu_amd as kf
from kungfu_amd.gguf import GGUF
import gguf_writer as gw
import oracle

pytestmark = pytest.mark.gpu


def test_gguf_weights_through_the_backend(cuda, tmp_path):
    n, n_out = 4096, 384
    mats = {}
    tensors = []
    for name, ty in (("blk.0.ffn_gate.weight", kf.TYPE_Q4_K), ("output.weight", kf.TYPE_Q6_K), ("blk.0.attn_q.weight", kf.TYPE_Q8_0)):
        w = kf.quantize(ty, kf.synth_normal(ty, 0.02, n * n_out).reshape(n_out, n))
        mats[name] = (ty, w)
        tensors.append((name, [n, n_out], ty, w.tobytes()))
    norm = kf.synth_normal(9, 1.0, n)
    tensors.append(("blk.0.attn_norm.weight", [n], 0, norm.tobytes()))
    path = tmp_path / "synthetic-q4_k_m.gguf"
    gw.write(path, [("general.architecture", "str", "llama"), ("llama.embedding_length", "u32", n)], tensors)

    x = kf.synth_normal(10, 1.0, 3 * n).reshape(3, n)
    with GGUF(path) as g:
        assert g.meta["llama.embedding_length"] == n
        assert np.array_equal(np.frombuffer(g.data("blk.0.attn_norm.weight").tobytes(), np.float32), norm)
        be = kf.Backend(0)
        try:
            for name, (ty, w) in mats.items():
                t = g.tensor(name)
                assert t.dims == (n, n_out) and t.ggml_type == ty
                data = g.data(name)
                wid = be.add_weight(t.ggml_type, t.dims, data)
                for rows in (1, 3):
                    got = be.matmul(wid, x[:rows], n_out)
                    want = oracle.matmul_slice(ty, np.array(data).reshape(n_out, -1), n, n_out, x[:rows])
                    err = np.abs(got - want)
                    assert (err <= 1e-4 + 1e-3 * np.abs(want)).all(), (name, rows, err.max())
        finally:
            be.close()
