"""CPU checks of the product library: it loads, exports every symbol include/kf_hip.h declares, validates arguments
before touching a GPU, and its host encoders / synthetic data match the oracle and their definitions."""
import ctypes
import json
import os

import numpy as np
import pytest

import kungfu_amd as kf
import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_library_exports_every_declared_symbol():
    L = kf.lib()
    syms = kf.declared_symbols()
    assert len(syms) >= 15
    for s in syms:
        assert hasattr(L, s), s
    assert L.kf_hip_abi_version() == 2


def test_knobs_read_once_from_the_environment_then_only_through_the_setter():
    """The launch knobs come from KF_* variables once per process (a flag knob by presence, a value knob by its
    integer); later environment changes are not seen, kf_hip_set_knob is. Runs in a fresh process."""
    import subprocess
    import sys

    code = (
        "import os, kungfu_amd as kf\n"
        "assert kf.get_knob('KF_GEMM_NO_TAIL') == 1 and kf.get_knob('KF_GEMV_MAXIT') == 3\n"
        "assert kf.get_knob('KF_GEMM_SK') == -1\n"
        "os.environ['KF_GEMM_SK'] = '1'\n"
        "assert kf.get_knob('KF_GEMM_SK') == -1\n"
        "kf.set_knob('KF_GEMM_SK', 0); assert kf.get_knob('KF_GEMM_SK') == 0\n"
        "kf.set_knob('KF_GEMM_NO_TAIL', None); assert kf.get_knob('KF_GEMM_NO_TAIL') == -1\n"
        "kf.set_knob('KF_GEMM_NO_TAIL', True); assert kf.get_knob('KF_GEMM_NO_TAIL') == 1\n"
        "try:\n    kf.set_knob('KF_NOT_A_KNOB', 1)\nexcept kf.KfError:\n    pass\nelse:\n    raise SystemExit(1)\n"
        "print('ok')\n"
    )
    env = dict(os.environ, KF_GEMM_NO_TAIL="0", KF_GEMV_MAXIT="3")
    env.pop("KF_GEMM_SK", None)
    r = subprocess.run([sys.executable, "-c", code], env=env, cwd=os.path.dirname(GOLDEN) + "/..", capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stderr


def test_act_layout_sections_are_aligned_and_sized():
    for rows, n in [(1, 4096), (3, 14336), (64, 256), (2048, 4096)]:
        o = kf.act_offsets(rows, n)
        total = kf.act_bytes(rows, n)
        assert all(v % 256 == 0 for v in o) and total % 256 == 0
        assert o[0] == 0 and o[1] >= rows * n and o[2] >= o[1] + rows * n // 16 * 4
        assert o[3] >= o[2] + rows * n // 16 * 4 and o[4] >= o[3] + rows * n // 32 * 4
        assert o[5] >= o[4] + rows * n // 32 * 4 and total >= o[5] + rows * ((n + 255) // 256) * 32


def test_act_kind_pairs_weight_types():
    assert kf.act_kind(kf.TYPE_Q8_0) == kf.ACT_Q8_0
    assert kf.act_kind(kf.TYPE_Q4_K) == kf.ACT_Q8K
    assert kf.act_kind(kf.TYPE_Q6_K) == kf.ACT_Q8K
    with pytest.raises(kf.KfError) as e:
        kf.act_kind(2)
    assert e.value.code == kf.KF_E_UNSUPPORTED and "2" in str(e.value)


FAKE = 0x10000  # a 256-byte aligned address the checks must reject before any HIP call


@pytest.mark.parametrize(
    "args,code,needle",
    [
        ((kf.TYPE_Q8_0, FAKE, kf.row_bytes(8, 4096), FAKE, None, None, FAKE, 1, 4096, 16, None), 0, None),
        ((2, FAKE, 100, FAKE, None, None, FAKE, 1, 4096, 16, None), kf.KF_E_UNSUPPORTED, "type 2"),
        ((kf.TYPE_Q4_K, FAKE, 144, FAKE, None, None, FAKE, 1, 200, 16, None), kf.KF_E_INVALID, "200 columns"),
        ((kf.TYPE_Q4_K, FAKE, 100, FAKE, None, None, FAKE, 1, 256, 16, None), kf.KF_E_INVALID, "row_bytes"),
        ((kf.TYPE_Q4_K, FAKE + 4, 144, FAKE, None, None, FAKE, 1, 256, 16, None), kf.KF_E_INVALID, "16-byte"),
        ((kf.TYPE_Q4_K, FAKE, 144, FAKE + 16, None, None, FAKE, 1, 256, 16, None), kf.KF_E_INVALID, "256-byte"),
        ((kf.TYPE_Q4_K, None, 144, FAKE, None, None, FAKE, 1, 256, 16, None), kf.KF_E_INVALID, "null"),
        ((kf.TYPE_Q4_K, FAKE, 144, FAKE, None, None, FAKE, 0, 256, 16, None), kf.KF_E_INVALID, "0 activation rows"),
        ((kf.TYPE_Q4_K, FAKE, 144 * 256, FAKE, None, None, FAKE, 1, 65536, 16, None), kf.KF_E_UNSUPPORTED, "LDS"),
    ],
)
def test_gemv_argument_checks(args, code, needle):
    if code == 0:
        return  # the valid row is only a template for the invalid ones (running it needs a GPU)
    rc = kf.lib().kf_hip_gemv(*args)
    assert rc == code
    assert needle in kf.last_error()


def test_quant_act_argument_checks():
    L = kf.lib()
    assert L.kf_hip_quant_act(FAKE, FAKE, 1, 4096, 5, None) == kf.KF_E_UNSUPPORTED
    assert L.kf_hip_quant_act(FAKE, FAKE, 1, 4016, 3, None) == kf.KF_E_INVALID
    assert L.kf_hip_quant_act(FAKE, FAKE, 1, 4096 + 32, 4, None) == kf.KF_E_INVALID
    assert L.kf_hip_quant_act(FAKE + 4, FAKE, 1, 4096, 4, None) == kf.KF_E_INVALID
    assert L.kf_hip_quant_act(None, FAKE, 1, 4096, 4, None) == kf.KF_E_INVALID
    assert L.kf_hip_matmul(kf.TYPE_Q4_K, FAKE, 4096 + 32, 8, FAKE, 1, FAKE, None, None, FAKE, None) == kf.KF_E_INVALID


def test_stream_read_argument_checks():
    """The read probe's checks run before any device call: null, misaligned, ragged or oversized buffers and an
    unsupported per-thread count are refused."""
    L = kf.lib()
    assert L.kf_hip_stream_read(None, 4096, 8, FAKE, None) == kf.KF_E_INVALID
    assert L.kf_hip_stream_read(FAKE, 4096, 8, None, None) == kf.KF_E_INVALID
    assert L.kf_hip_stream_read(FAKE + 8, 4096, 8, FAKE, None) == kf.KF_E_INVALID
    assert "misaligned" in kf.last_error()
    assert L.kf_hip_stream_read(FAKE, 4100, 8, FAKE, None) == kf.KF_E_INVALID
    assert L.kf_hip_stream_read(FAKE, 0, 8, FAKE, None) == kf.KF_E_INVALID
    assert L.kf_hip_stream_read(FAKE, 1 << 36, 8, FAKE, None) == kf.KF_E_INVALID
    assert L.kf_hip_stream_read(FAKE, 4096, 6, FAKE, None) == kf.KF_E_INVALID
    assert "pieces a thread" in kf.last_error()


def test_backend_errors_without_a_device():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    L = kf.lib()
    assert L.kf_hip_backend_new(0) is None
    assert "device 0" in kf.last_error()
    assert L.kf_hip_backend_matmul(None, 0, None, 1, 4, None, None) == kf.KF_E_INVALID


def test_quantize_q8_0_matches_oracle():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((6, 1024)) * rng.uniform(1e-3, 10, (6, 1))).astype(np.float32)
    x[2, :64] = 0.0
    x[3, 5] = 1e30
    assert np.array_equal(kf.quantize(kf.TYPE_Q8_0, x), oracle.q8_0_quantize(x))


def test_quantize_q4_k_round_trip():
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((4, 1024)) * 0.02).astype(np.float32)
    x[1, :256] = 0.0
    x[2, :256] = np.abs(x[2, :256])  # all-positive super-block: min 0
    w = kf.quantize(kf.TYPE_Q4_K, x)
    deq = oracle.dequant(12, w, 1024)
    assert not deq[1, :256].any()
    for r in range(4):
        blk = w[r].reshape(-1, 144)
        for b in range(4):
            d = float(blk[b, 0:2].copy().view(np.float16)[0])
            dmin = float(blk[b, 2:4].copy().view(np.float16)[0])
            xs = x[r, 256 * b : 256 * (b + 1)].reshape(8, 32)
            err = np.abs(deq[r, 256 * b : 256 * (b + 1)].reshape(8, 32) - xs)
            # per sub-block: half a step of its scale plus the rounding of its min, and the 6-bit scale rounding
            step = (xs.max(axis=1) - np.minimum(xs.min(axis=1), 0)) / 15
            assert (err.max(axis=1) <= 0.5 * step + 0.5 * d + 0.5 * dmin + 32 * d + 1e-7).all()
        rel = np.sqrt(((deq[r] - x[r]) ** 2).mean()) / np.sqrt((x[r] ** 2).mean() + 1e-30)
        if r != 1:
            assert rel < 0.12


def test_quantize_q5_k_and_q6_k_round_trip():
    """The library's q5_K / q6_K encoders read back through the oracle's dequant (pinned to ggml's fixtures): errors
    within half a quantization step plus the scale roundings, zeros exact, and the expected RMS ordering."""
    rng = np.random.default_rng(13)
    x = (rng.standard_normal((4, 1024)) * 0.02).astype(np.float32)
    x[1, :256] = 0.0
    rel = {}
    for ty, size in ((kf.TYPE_Q5_K, 176), (kf.TYPE_Q6_K, 210)):
        w = kf.quantize(ty, x)
        assert w.shape == (4, 4 * size)
        deq = oracle.dequant(ty, w, 1024)
        assert not deq[1, :256].any()
        for r in range(4):
            blk = w[r].reshape(-1, size)
            for b in range(4):
                xs = x[r, 256 * b : 256 * (b + 1)]
                err = np.abs(deq[r, 256 * b : 256 * (b + 1)] - xs)
                if ty == kf.TYPE_Q6_K:
                    d = float(blk[b, 208:210].copy().view(np.float16)[0])
                    g = xs.reshape(16, 16)
                    # per 16: half a step of amax / 31, plus the int8 scale rounding (half of d) over 31 steps
                    step = np.abs(g).max(axis=1) / 31
                    assert (err.reshape(16, 16).max(axis=1) <= 0.5 * step + 31 * 0.5 * d + 1e-7).all()
                else:
                    d = float(blk[b, 0:2].copy().view(np.float16)[0])
                    dmin = float(blk[b, 2:4].copy().view(np.float16)[0])
                    g = xs.reshape(8, 32)
                    step = (g.max(axis=1) - np.minimum(g.min(axis=1), 0)) / 31
                    assert (err.reshape(8, 32).max(axis=1) <= 0.5 * step + 0.5 * d + 0.5 * dmin + 64 * d + 1e-7).all()
        rel[ty] = np.sqrt(((deq - x) ** 2).mean() / (x ** 2).mean())
    q4 = oracle.dequant(12, kf.quantize(kf.TYPE_Q4_K, x), 1024)
    assert rel[kf.TYPE_Q6_K] < rel[kf.TYPE_Q5_K] < np.sqrt(((q4 - x) ** 2).mean() / (x ** 2).mean())


def test_k_quant_types_take_the_k_product_and_the_gemm_where_aligned():
    L = kf.lib()
    assert kf.act_kind(kf.TYPE_Q5_K) == kf.ACT_Q8K and kf.act_kind(kf.TYPE_Q6_K) == kf.ACT_Q8K
    # the q6_K GEMM needs rows that start 16-byte aligned (2304 columns: 9 x 210 bytes a row)
    rc = L.kf_hip_gemm_i8(kf.TYPE_Q6_K, FAKE, kf.row_bytes(14, 2304), FAKE, None, None, FAKE, 64, 2304, 16, None)
    assert rc == kf.KF_E_UNSUPPORTED and "kf_hip_gemv" in kf.last_error()
    rc = L.kf_hip_moe_gemv(kf.TYPE_Q5_K, FAKE, None, kf.row_bytes(13, 4096) * 16, kf.row_bytes(13, 4096), FAKE, 1, 4096, 16,
                           FAKE, FAKE, 1, 1, 0, FAKE, None)
    assert rc == kf.KF_E_UNSUPPORTED and "q8_0 and q4_K" in kf.last_error()
    rc = L.kf_hip_gemv(kf.TYPE_Q6_K, FAKE, kf.row_bytes(14, 4096) + 2, FAKE, None, None, FAKE, 1, 4096, 16, None)
    assert rc == kf.KF_E_INVALID and "row_bytes" in kf.last_error()


def _synth_numpy(seed, sigma, n):
    """SplitMix64 then Box-Muller in double: z0 = r cos(2 pi u2), z1 = r sin(2 pi u2), r = sqrt(-2 ln u1),
    u = ((next >> 11) + 0.5) * 2^-53, output f32(sigma * r * trig)."""
    M = (1 << 64) - 1
    s = seed
    out = np.empty(n, np.float32)

    def nxt():
        nonlocal s
        s = (s + 0x9E3779B97F4A7C15) & M
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        return z ^ (z >> 31)

    for i in range(0, n, 2):
        u1 = ((nxt() >> 11) + 0.5) * 2.0**-53
        u2 = ((nxt() >> 11) + 0.5) * 2.0**-53
        r = np.sqrt(-2.0 * np.log(u1))
        out[i] = np.float32(sigma * r * np.cos(2 * np.pi * u2))
        if i + 1 < n:
            out[i + 1] = np.float32(sigma * r * np.sin(2 * np.pi * u2))
    return out


def test_synth_normal_matches_definition_and_golden():
    got = kf.synth_normal(0, 1.0, 1001)
    want = _synth_numpy(0, 1.0, 1001)
    assert np.abs(got.astype(np.float64) - want).max() <= 2e-7 * np.abs(want).max()
    gold = json.load(open(os.path.join(GOLDEN, "synth_normal_seed0.json")))
    assert np.array_equal(np.array(gold["bits"], np.uint32), got[:64].view(np.uint32))
    big = kf.synth_normal(1, 0.02, 200000)
    assert abs(big.mean()) < 3e-4 and abs(big.std() - 0.02) < 2e-4


def test_group_segment_table_is_validated_on_the_host():
    """kf_hip_gemv_group / kf_hip_matmul_group reject a bad segment table before any launch."""
    L = kf.lib()
    N = kf.SEG_NONE

    def run(words, nseg=None, w=FAKE):
        a = np.asarray(words, dtype=np.int64)
        rc = L.kf_hip_gemv_group(kf.TYPE_Q4_K, w, 144, FAKE, FAKE, 1, 256, a.ctypes.data if len(a) else None,
                                 len(a) // 6 if nseg is None else nseg, None)
        return rc, L.kf_hip_last_error().decode()

    good = [0, 0, N, N, 0, 16, 144 * 16, 64, N, N, 16, 8]
    assert run([], 0)[0] == kf.KF_E_INVALID
    assert run(good * 3, 5)[0] == kf.KF_E_INVALID                         # above four members
    rc, msg = run([0, 0, N, N, 0, 16, 144 * 16, 64, N, N, 17, 8])          # a gap in the stacking
    assert rc == kf.KF_E_INVALID and "starts at row 17" in msg
    rc, msg = run([0, 0, N, N, 0, 16, 8, 64, N, N, 16, 8])                 # member weights not 16-byte aligned
    assert rc == kf.KF_E_INVALID and "16-byte" in msg
    rc, msg = run([0, 0, N, N, 0, 16, N, 64, N, N, 16, 8])                 # no weights
    assert rc == kf.KF_E_INVALID and "no weights" in msg
    rc, msg = run([0, 0, N, N, 0, 0])                                      # an empty member
    assert rc == kf.KF_E_INVALID and "0 rows" in msg
    rc, msg = run([0, 0, 2, N, 0, 16])                                     # a misaligned bias
    assert rc == kf.KF_E_INVALID and "4-byte" in msg
    rc = L.kf_hip_matmul_group(kf.TYPE_Q4_K, FAKE, 200, FAKE, 1, FAKE, FAKE, np.asarray(good, np.int64).ctypes.data, 2, None)
    assert rc == kf.KF_E_INVALID and "200 columns" in L.kf_hip_last_error().decode()
    rc = L.kf_hip_matmul_group(2, FAKE, 256, FAKE, 1, FAKE, FAKE, np.asarray(good, np.int64).ctypes.data, 2, None)
    assert rc == kf.KF_E_UNSUPPORTED
